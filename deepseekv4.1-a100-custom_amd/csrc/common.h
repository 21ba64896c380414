// Shared device helpers of the MI355X (gfx950) FP4 MoE expert path.
//
// Formats (the reference's quant.py:6-110):
//   E2M1 weights, two per byte along k, low nibble = even k; one E8M0 byte per (row, 32 k), value 2^(b-127).
//   FP8 activations: E4M3 (float8_e4m3fn) codes with one E8M0 byte per 32 k (power-of-two scale).
// The rounding helpers are integer/bit based, or (FP8 encode and decode) the gfx950 conversion instructions checked
// bit for bit against them, so results do not depend on the FP mode (denormal flush).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dsv41_amd.h"  // the C ABI: definitions below must match these declarations

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

#define DSV41_EINVAL (-1)
#define DSV41_ENOSPACE (-2)   // the no-allocation entry point's scratch array is too small for the call

#define WAVE 64

// ------------------------------------------------------------------------------------------ bf16
__device__ __forceinline__ float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// fp32 -> bf16 bits, round to nearest even; every NaN becomes 0xFFFF (torch's vectorised CPU conversion)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0xFFFFu;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16_bits(f)); }

// ------------------------------------------------------------------------------------------ E2M1 x E8M0
// Exact fp32 bit pattern of E2M1 code c times 2^(b-127), as quant.dequant_fp4 computes it in fp32
// (quant.py:106-110): byte 0 is the subnormal 2^-127, 255 is +inf (so 0 x inf = NaN). Built from integers:
// |value| = M * 2^(b-128) with M = 2|v| in {0,1,2,3,4,6,8,12}.
__device__ __forceinline__ uint32_t e2m1_e8m0_f32_bits(uint32_t c, uint32_t b) {
    const uint32_t sign = (c & 8u) << 28;
    const uint32_t mag = c & 7u;
    const uint32_t M = (mag < 2u) ? mag : ((2u | (mag & 1u)) << ((mag >> 1) - 1u));
    if (b == 255u) return M ? (sign | 0x7F800000u) : 0xFFC00000u;
    if (M == 0u) return sign;
    const uint32_t h = 31u - __builtin_clz(M);            // 0..3
    const int biased = (int)h + (int)b - 1;                // biased fp32 exponent of M * 2^(b-128)
    if (biased >= 255) return sign | 0x7F800000u;
    if (biased >= 1) return sign | ((uint32_t)biased << 23) | ((M << (23u - h)) & 0x7FFFFFu);
    return sign | (M << (b + 21u));                        // subnormal: M * 2^(b-128) / 2^-149
}

// E8M0 byte -> fp32 2^(b-127) bit pattern (quant.py:27-31): 0 -> 2^-127 (subnormal), 255 -> +inf
__device__ __forceinline__ float e8m0_to_f32(uint32_t b) { return __uint_as_float(b ? (b << 23) : 0x00400000u); }

// ------------------------------------------------------------------------------------------ E4M3 (fp8)
// Round |v| <= 448 to the float8_e4m3fn grid, ties to even, sign kept (-0.0 stays -0.0 as in torch's cast,
// quant.py:53; the explicit formula is fused.py:24-34). The ulp is a power of two, so v * 2^(3-e) is exact.
__device__ __forceinline__ float round_e4m3(float v) {
    const float a = fabsf(v);
    int e = (int)((__float_as_uint(a) >> 23) & 0xFFu) - 127;
    e = e < -6 ? -6 : e;
    const float inv_ulp = __uint_as_float((uint32_t)(127 + 3 - e) << 23);
    const float ulp = __uint_as_float((uint32_t)(127 - 3 + e) << 23);
    float r = rintf(a * inv_ulp) * ulp;
    r = fminf(r, 448.0f);
    return __uint_as_float(__float_as_uint(r) | (__float_as_uint(v) & 0x80000000u));
}

// float8_e4m3fn bits of a value already on the E4M3 grid
__device__ __forceinline__ uint32_t e4m3_encode(float q) {
    const uint32_t u = __float_as_uint(q);
    const uint32_t s = (u >> 24) & 0x80u;
    const float a = __uint_as_float(u & 0x7FFFFFFFu);
    uint32_t code;
    if (a >= 0.015625f) code = ((((u >> 23) & 0xFFu) - 120u) << 3) | ((u >> 20) & 7u);
    else code = (uint32_t)(a * 512.0f);                  // subnormal grid: multiples of 2^-9 (exact)
    return s | code;
}

__device__ __forceinline__ float e4m3_decode(uint32_t c) {
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    const float mag = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0.001953125f;
    return (c & 0x80u) ? -mag : mag;
}

// Per-32 FP8 block quantisation (quant.py:45-64; fused.py:47-69 MODE 0): given the group's amax, the
// power-of-two exponent e (scale 2^e, E8M0 byte e + 127). amax is clamped to >= 1e-4 and divided by 448
// with an IEEE division, then ceil(log2) exactly from the bits (fused.py:10-16).
__device__ __forceinline__ int fq8_exponent(float amax) {
    const float r = fmaxf(amax, 1e-4f) / 448.0f;
    const uint32_t u = __float_as_uint(r);
    return (int)((u >> 23) & 0xFFu) - 127 + ((u & 0x7FFFFFu) != 0u ? 1 : 0);
}

// v / 2^e clamped to +-448 (the division by a power of two is exact; a NaN v becomes -448, as fmaxf drops it)
__device__ __forceinline__ float fq8_scaled(float v, int e) {
    return fminf(fmaxf(v * __uint_as_float((uint32_t)(127 - e) << 23), -448.0f), 448.0f);
}

// code of v at scale 2^e: RNE_e4m3(clamp(v / 2^e, +-448)), by arithmetic on the bits
__device__ __forceinline__ uint32_t fq8_code_sw(float v, int e) { return e4m3_encode(round_e4m3(fq8_scaled(v, e))); }

// The same codes from the hardware conversion: v_cvt_pk_fp8_f32 rounds two fp32 values to nearest even on the
// float8_e4m3fn grid (subnormals included) and packs them into bits 0-15 of a word (or 16-31 with hi). Every input
// is clamped to +-448 first, so no conversion leaves the grid. Bit-identical with fq8_code_sw: the self-test entry
// dsv41_selftest_fp8_cvt compares the two over every bf16 value, every rounding midpoint and random fp32 inputs.
__device__ __forceinline__ uint32_t fq8_code2_hw(float a, float b, int e) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fq8_scaled(a, e), fq8_scaled(b, e), 0, false) & 0xFFFFu;
}
__device__ __forceinline__ uint32_t fq8_code4_hw(float a, float b, float c, float d, int e) {
    const int w = __builtin_amdgcn_cvt_pk_fp8_f32(fq8_scaled(a, e), fq8_scaled(b, e), 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fq8_scaled(c, e), fq8_scaled(d, e), w, true);
}
__device__ __forceinline__ uint32_t fq8_code_hw(float v, int e) { return fq8_code2_hw(v, v, e) & 0xFFu; }

__device__ __forceinline__ uint32_t fq8_code(float v, int e) { return fq8_code_hw(v, e); }

__device__ __forceinline__ float fq8_value(uint32_t code, int e) {
    return e4m3_decode(code) * __uint_as_float((uint32_t)(127 + e) << 23);
}

// byte B of a word of E4M3 codes (a code fq8 produces: never the NaN codes 0x7F / 0xFF) as fp32, by the hardware
// conversion (v_cvt_f32_fp8), times 2^e
template <int B>
__device__ __forceinline__ float fq8_value_hw(uint32_t word, int e) {
    return __builtin_amdgcn_cvt_f32_fp8((int)word, B) * __uint_as_float((uint32_t)(127 + e) << 23);
}

// ------------------------------------------------------------------------------------------ two-term FP8 split
// bf16 activations off the FP8 grid as two E4M3 x E8M0 terms per 32-group: hi = the per-32 rounding above, lo = the
// residual x - hi (exact in fp32: x has 8 significant bits, hi 4, within 24 bits of each other) rounded the same way
// with a scale of its own. hi + lo == x unless a residual falls below lo's normal range (then within 2^-21 of the
// group's amax). lo's exponent: the smallest e >= -126 with amax / 2^e <= 448, no floor (residuals may be tiny):
// amax = m 2^ea, m in [1, 2), needs 2^e >= m / 1.75 * 2^(ea - 8), i.e. e = ea - 8 when m <= 1.75, else ea - 7.
__device__ __forceinline__ int lo_exponent(float amax) {
    const uint32_t u = __float_as_uint(amax);
    const int ea = (int)((u >> 23) & 0xFFu) - 127;
    if (ea < -126) return -126;                           // zero or subnormal: 448 * 2^-126 exceeds it
    const int e = ea - 8 + ((u & 0x7FFFFFu) > 0x600000u ? 1 : 0);
    return e < -126 ? -126 : e;
}

// One lane's 16 consecutive bf16 values (two 16-byte vectors) of a 32-group whose other half sits on the adjacent
// lane (lane ^ 1, which must run the same call): their hi and lo codes as 16 bytes each, in natural k order when the
// input is 8-k permuted (position j holds input position (j & ~7) | bitrev3(j & 7)), and the two exponents (E8M0
// bytes e + 127). Returns whether a lo code of this lane is non-zero.
__device__ __forceinline__ bool fp8_split16(const v4i w0, const v4i w1, int permuted, v4i& hi, v4i& lo, int& e, int& e2) {
    const uint32_t wd[8] = {(uint32_t)w0.x, (uint32_t)w0.y, (uint32_t)w0.z, (uint32_t)w0.w,
                            (uint32_t)w1.x, (uint32_t)w1.y, (uint32_t)w1.z, (uint32_t)w1.w};
    // value at input position i (bf16 -> fp32 is a shift)
    auto val = [&](int i) { return __uint_as_float((i & 1) ? (wd[i >> 1] & 0xFFFF0000u) : (wd[i >> 1] << 16)); };
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(val(i)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 2));
    e = fq8_exponent(amax);
    // codes in output (natural k) order: position j holds input position (j & ~7) | bitrev3(j & 7) when permuted; four
    // codes per conversion pair, the residuals from the codes' decoded values (only their amax depends on all of them)
    float v[16], r[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int sj = (j & ~7) | ((j & 1) << 2) | (j & 2) | ((j >> 2) & 1);
        v[j] = permuted ? val(sj) : val(j);
    }
    uint32_t cw[4], cw2[4];
    float rmax = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        cw[q] = fq8_code4_hw(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3], e);
        r[4 * q + 0] = __fsub_rn(v[4 * q + 0], fq8_value_hw<0>(cw[q], e));   // the residuals, exact
        r[4 * q + 1] = __fsub_rn(v[4 * q + 1], fq8_value_hw<1>(cw[q], e));
        r[4 * q + 2] = __fsub_rn(v[4 * q + 2], fq8_value_hw<2>(cw[q], e));
        r[4 * q + 3] = __fsub_rn(v[4 * q + 3], fq8_value_hw<3>(cw[q], e));
#pragma unroll
        for (int i = 0; i < 4; ++i) rmax = fmaxf(rmax, fabsf(r[4 * q + i]));
    }
    rmax = fmaxf(rmax, __shfl_xor(rmax, 1, 2));
    e2 = lo_exponent(rmax);
    uint32_t nz = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        cw2[q] = fq8_code4_hw(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3], e2);
        nz |= cw2[q] & 0x7F7F7F7Fu;
    }
    hi = v4i{(int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3]};
    lo = v4i{(int)cw2[0], (int)cw2[1], (int)cw2[2], (int)cw2[3]};
    return nz != 0;
}

// ------------------------------------------------------------------------------------------ waves
__device__ __forceinline__ float wave_max32(float v) {  // max over each 32-lane half of the wave
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 32));
    return v;
}

// Full-wave reductions on DPP row operations (a few cycles per step, no LDS crossbar round trips): the classic
// row_shr 1/2/3, row_shr 4/8 (bank masked), row_bcast 15/31 sequence leaves the result in lane 63, which
// readlane broadcasts. Lanes a DPP step has no source for keep their own value (update_dpp with old = self).
#define DPP_STEP(T, x, op, ctrl, rmask, bmask)                                                                 \
    x = op(x, __builtin_bit_cast(T, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, x),                    \
                                                                __builtin_bit_cast(int, x), ctrl, rmask, bmask, false)))
__device__ __forceinline__ float fmax2(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ float fadd2(float a, float b) { return a + b; }

__device__ __forceinline__ float wave_reduce_max(float x) {
    DPP_STEP(float, x, fmax2, 0x111, 0xF, 0xF);   // row_shr:1
    DPP_STEP(float, x, fmax2, 0x112, 0xF, 0xF);   // row_shr:2
    DPP_STEP(float, x, fmax2, 0x113, 0xF, 0xF);   // row_shr:3
    DPP_STEP(float, x, fmax2, 0x114, 0xF, 0xE);   // row_shr:4
    DPP_STEP(float, x, fmax2, 0x118, 0xF, 0xC);   // row_shr:8
    DPP_STEP(float, x, fmax2, 0x142, 0xA, 0xF);   // row_bcast:15
    DPP_STEP(float, x, fmax2, 0x143, 0xC, 0xF);   // row_bcast:31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// wave sum in a fixed order (the same DPP tree every call): deterministic. Steps 1-3 add the ORIGINAL values of
// lanes i-1, i-2, i-3 (a running source would count elements twice); steps 4-7 combine partial sums. Lanes a
// step has no source for add 0 (update_dpp with old = 0).
__device__ __forceinline__ float wave_reduce_sum(float x) {
#define DPP_SRC(v, ctrl, rmask, bmask) \
    __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), ctrl, rmask, bmask, false))
    float t = x;
    t += DPP_SRC(x, 0x111, 0xF, 0xF);   // row_shr:1
    t += DPP_SRC(x, 0x112, 0xF, 0xF);   // row_shr:2
    t += DPP_SRC(x, 0x113, 0xF, 0xF);   // row_shr:3
    t += DPP_SRC(t, 0x114, 0xF, 0xE);   // row_shr:4, lanes 4..15 of each row
    t += DPP_SRC(t, 0x118, 0xF, 0xC);   // row_shr:8, lanes 8..15
    t += DPP_SRC(t, 0x142, 0xA, 0xF);   // row_bcast:15 into rows 1, 3
    t += DPP_SRC(t, 0x143, 0xC, 0xF);   // row_bcast:31 into rows 2, 3
#undef DPP_SRC
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), 63));
}

__device__ __forceinline__ unsigned umax2(unsigned a, unsigned b) { return a > b ? a : b; }
__device__ __forceinline__ unsigned wave_reduce_max_u32(unsigned x) {
    DPP_STEP(unsigned, x, umax2, 0x111, 0xF, 0xF);
    DPP_STEP(unsigned, x, umax2, 0x112, 0xF, 0xF);
    DPP_STEP(unsigned, x, umax2, 0x113, 0xF, 0xF);
    DPP_STEP(unsigned, x, umax2, 0x114, 0xF, 0xE);
    DPP_STEP(unsigned, x, umax2, 0x118, 0xF, 0xC);
    DPP_STEP(unsigned, x, umax2, 0x142, 0xA, 0xF);
    DPP_STEP(unsigned, x, umax2, 0x143, 0xC, 0xF);
    return (unsigned)__builtin_amdgcn_readlane((int)x, 63);
}

// wave max of unsigned values whose identity is 0: a DPP source lane that does not exist or a row the mask
// leaves out reads 0 (old = 0, bound_ctrl), which lets the compiler fold each move into the max
__device__ __forceinline__ unsigned wave_reduce_max_u32z(unsigned x) {
#define DPP_MAXZ(ctrl, rmask, bmask) x = umax2(x, (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, ctrl, rmask, bmask, true))
    DPP_MAXZ(0x111, 0xF, 0xF);   // row_shr:1
    DPP_MAXZ(0x112, 0xF, 0xF);   // row_shr:2
    DPP_MAXZ(0x114, 0xF, 0xF);   // row_shr:4 (after shr 1, 2: lane i holds lanes i-3..i)
    DPP_MAXZ(0x118, 0xF, 0xF);   // row_shr:8
    DPP_MAXZ(0x142, 0xA, 0xF);   // row_bcast:15 into rows 1, 3
    DPP_MAXZ(0x143, 0xC, 0xF);   // row_bcast:31 into rows 2, 3
#undef DPP_MAXZ
    return (unsigned)__builtin_amdgcn_readlane((int)x, 63);
}

// wave max of 64-bit unsigned keys (two 32-bit DPP moves per step)
__device__ __forceinline__ unsigned long long wave_reduce_max_u64(unsigned long long x) {
#define DPP_MAX64(ctrl, rmask, bmask)                                                                          \
    {                                                                                                          \
        const unsigned lo = (unsigned)x, hi = (unsigned)(x >> 32);                                             \
        const unsigned nlo = (unsigned)__builtin_amdgcn_update_dpp((int)lo, (int)lo, ctrl, rmask, bmask, false); \
        const unsigned nhi = (unsigned)__builtin_amdgcn_update_dpp((int)hi, (int)hi, ctrl, rmask, bmask, false); \
        const unsigned long long n = ((unsigned long long)nhi << 32) | nlo;                                    \
        x = n > x ? n : x;                                                                                     \
    }
    DPP_MAX64(0x111, 0xF, 0xF);
    DPP_MAX64(0x112, 0xF, 0xF);
    DPP_MAX64(0x113, 0xF, 0xF);
    DPP_MAX64(0x114, 0xF, 0xE);
    DPP_MAX64(0x118, 0xF, 0xC);
    DPP_MAX64(0x142, 0xA, 0xF);
    DPP_MAX64(0x143, 0xC, 0xF);
#undef DPP_MAX64
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)x, 63);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(x >> 32), 63);
    return ((unsigned long long)hi << 32) | lo;
}

// float -> uint32 whose unsigned order is the float order (NaN excluded by the caller)
__device__ __forceinline__ unsigned float_order_key(float f) {
    const unsigned u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ------------------------------------------------------------------------------------------ MFMA
// D(16x16, fp32) += A(16x128) * B(128x16) with per-32 E8M0 block scales (gfx950 block-scaled MFMA).
// Lane layouts (measured on gfx950 by tests/test_gpu_mfma_layout.py), g = l/16:
// A = E2M1 weights (format 4): lane l holds row l%16, k [32g, 32g+32) contiguous: 16 bytes in the low 4 dwords,
//     low nibble first. B = E4M3 activations (format 0): lane l holds column l%16, bytes 0-15 = k [16g, 16g+16)
//     and bytes 16-31 = k [64+16g, 64+16g+16). sa / sb: byte 0 of the lane's register, the E8M0 scale of
//     32-k block g of row / column l%16. Output: lane l holds D[4g+i][l%16], i = 0..3.
__device__ __forceinline__ v4f mfma_fp4w_fp8x(v8i a, v8i b, v4f c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 0, 0, sa, 0, sb);
}
// The same with the two E8M0 bytes taken from byte ja of sa and byte jb of sb (the instruction's scale byte selects;
// ja, jb must fold to constants 0..3)
template <int JA, int JB>
__device__ __forceinline__ v4f mfma_fp4w_fp8x_b(v8i a, v8i b, v4f c, int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 4, 0, JA, sa, JB, sb);
}
__device__ __forceinline__ v4f mfma_fp4w_fp8x_sel(int ja, int jb, v8i a, v8i b, v4f c, int sa, int sb) {
#define MFMA_SEL(A, B) case (A) * 4 + (B): return mfma_fp4w_fp8x_b<A, B>(a, b, c, sa, sb);
    switch (ja * 4 + jb) {
        MFMA_SEL(0, 0) MFMA_SEL(0, 1) MFMA_SEL(0, 2) MFMA_SEL(0, 3) MFMA_SEL(1, 0) MFMA_SEL(1, 1) MFMA_SEL(1, 2) MFMA_SEL(1, 3)
        MFMA_SEL(2, 0) MFMA_SEL(2, 1) MFMA_SEL(2, 2) MFMA_SEL(2, 3) MFMA_SEL(3, 0) MFMA_SEL(3, 1) MFMA_SEL(3, 2)
        default: return mfma_fp4w_fp8x_b<3, 3>(a, b, c, sa, sb);
    }
#undef MFMA_SEL
}

// ------------------------------------------------------------------------------------------ weight tiles
// Byte offset of lane `lane`'s 16 weight bytes for 16-row block nb, k-chunk kc (128 k), and of its scale byte.
// Lane l: row nb*16 + l%16, k [kc*128 + 32*(l/16), +32).
template <int TILED>
__device__ __forceinline__ long long wtile_off(int nb, int kc, int nk, int Kh, int lane) {
    if (TILED) return ((long long)nb * nk + kc) * 1024 + (lane & 15) * 64 + (lane >> 4) * 16;   // quant.py:118-122
    return ((long long)nb * 16 + (lane & 15)) * Kh + kc * 64 + (lane >> 4) * 16;
}
template <int TILED>
__device__ __forceinline__ long long stile_off(int nb, int kc, int nk, int Ks, int lane) {
    if (TILED) return ((long long)nb * nk + kc) * 64 + (lane & 15) * 4 + (lane >> 4);           // quant.py:130-134
    return ((long long)nb * 16 + (lane & 15)) * Ks + kc * 4 + (lane >> 4);
}

// weight tiles are streamed once: non-temporal loads keep them from displacing reused data in the caches
#ifndef DSV41_WEIGHT_NT
#define DSV41_WEIGHT_NT 1
#endif
__device__ __forceinline__ v4i load_weight_tile(const uint8_t* p) {
#if DSV41_WEIGHT_NT
    return __builtin_nontemporal_load((const v4i*)p);
#else
    return *(const v4i*)p;
#endif
}
// Buffer loads: a 128-bit descriptor in scalar registers holds the base address and the byte count, the lane
// supplies a 32-bit offset and the loop a scalar one. Per-lane 64-bit addresses (two VGPRs per in-flight slot)
// disappear, and an offset at or beyond `bytes` reads 0 instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ v4i buffer_load_tile(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, DSV41_WEIGHT_NT ? 2 : 0));
}
__device__ __forceinline__ int buffer_load_byte(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (int)__builtin_amdgcn_raw_buffer_load_b8(r, voff, soff, 0);
}
// weight tiles in flight per wave in the grouped kernel with LDS-staged activation rows (decode-sized groups): 4 was
// faster and steadier than 6, 8, 12 or 16 on the configs[1] drop-in sequences (alternating builds on one box)
#ifndef DSV41_PF_UP
#define DSV41_PF_UP 4
#endif

// ------------------------------------------------------------------------------------------ E4M3 weights -> bf16 MFMA operands
typedef __bf16 v8bf16_t __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf16_t __attribute__((ext_vector_type(2)));

// 16 E4M3 bytes -> two bf16x8 MFMA operands (bytes 0..7, 8..15), each value times the scale `sc` (a power of two:
// E4M3 x 2^e has at most 4 significant bits, so the product is exact in bf16 over its normal range)
__device__ __forceinline__ void decode16(const v4i w, float sc, v8bf16_t& lo, v8bf16_t& hi) {
    const v2bf16_t p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)w.x, sc, false);
    const v2bf16_t p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)w.x, sc, true);
    const v2bf16_t p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)w.y, sc, false);
    const v2bf16_t p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)w.y, sc, true);
    const v2bf16_t q0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)w.z, sc, false);
    const v2bf16_t q1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)w.z, sc, true);
    const v2bf16_t q2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)w.w, sc, false);
    const v2bf16_t q3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((uint32_t)w.w, sc, true);
    lo = __builtin_shufflevector(__builtin_shufflevector(p0, p1, 0, 1, 2, 3), __builtin_shufflevector(p2, p3, 0, 1, 2, 3),
                                 0, 1, 2, 3, 4, 5, 6, 7);
    hi = __builtin_shufflevector(__builtin_shufflevector(q0, q1, 0, 1, 2, 3), __builtin_shufflevector(q2, q3, 0, 1, 2, 3),
                                 0, 1, 2, 3, 4, 5, 6, 7);
}

// ------------------------------------------------------------------------------------------ load pipeline
// Software pipeline over n iterations with PF register slots: load(slot, it) fills a slot, use(slot) consumes
// it. The steady-state loop has no guards (every load in bounds); only the peeled drain has uniform (scalar)
// guards, so the compiler can keep PF loads in flight with exact vmcnt waits instead of draining the queue.
template <int PF, typename LoadF>
__device__ __forceinline__ void pipeline_start(int n, LoadF&& load) {
    // unconditional prologue: the loop is entered with exactly PF slots in flight, in slot order, so the
    // waitcnt pass can wait for the oldest slot only (a conditional prologue makes it drain the queue);
    // sched_barrier(0) keeps each consume/refill pair in program order
    if (n < PF) return;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
        load(i, i);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// UNCOND: load(slot, it) is safe for it >= n (a buffer load past its descriptor's range returns 0 without a memory
// access), so the drain and the short path issue their loads unconditionally: each slot register is then written on
// every path and the compiler keeps no copies of the old value (a conditional load makes the slot a phi).
// DRAIN_BARRIER: a scheduling barrier after each consume of the drain and the short path too, so the compiler does not
// hoist every remaining slot's operand reads (LDS) ahead of the first MFMA and keeps them live together.
template <int PF, bool DRAIN_BARRIER = false, bool UNCOND = false, typename LoadF, typename UseF>
__device__ __forceinline__ void pipeline_finish(int n, LoadF&& load, UseF&& use) {
    if (n < PF) {  // short: issue every load, then consume in order (one memory latency, not n)
#pragma unroll
        for (int i = 0; i < PF; ++i)
            if (UNCOND || i < n) load(i, i);
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            if (i < n) use(i);
            if (DRAIN_BARRIER) __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
    int it = 0;
    for (; it + 2 * PF <= n; it += PF) {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            use(i);
            load(i, it + PF + i);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
        use(i);
        if (UNCOND || it + PF + i < n) load(i, it + PF + i);
        __builtin_amdgcn_sched_barrier(0);
    }
    it += PF;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
        if (it + i < n) use(i);
        if (DRAIN_BARRIER) __builtin_amdgcn_sched_barrier(0);
    }
}

template <int PF, typename LoadF, typename UseF>
__device__ __forceinline__ void pipelined(int n, LoadF&& load, UseF&& use) {
    pipeline_start<PF>(n, load);
    pipeline_finish<PF>(n, load, use);
}

// The same pipeline over a compile-time trip count NK, fully unrolled: straight-line code lets the waitcnt pass
// emit exact rolling waits (wait for the oldest slot only) instead of draining the queue at a loop head.
template <int PF, int NK, typename LoadF, typename UseF>
__device__ __forceinline__ void pipelined_fixed(LoadF&& load, UseF&& use) {
#pragma unroll
    for (int i = 0; i < (PF < NK ? PF : NK); ++i) load(i, i);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int it = 0; it < NK; ++it) {
        use(it % PF);
        if (it + PF < NK) load(it % PF, it + PF);
        __builtin_amdgcn_sched_barrier(0);
    }
}
