// Format kernels: E2M1 x E8M0 dequantisation (bit-exact with quant.dequant_fp4), per-32 FP8 block
// quantisation of activations (quant.quant_fp8 / fake_quant_fp8), and the SwiGLU epilogue that turns the
// fp32 gate/up GEMV output into FP8 codes for the down projection (fused.swiglu_quant).
// All are HBM-bound element-wise kernels: coalesced loads, one 32-lane half-wave per 32-element FP8 group.
#include "common.h"

// ------------------------------------------------------------------------------------------ dequant
// out[n, k] (bf16 bits) = E2M1(code of k in row n) * 2^(S[n, k/32] - 127) rounded to bf16 (quant.py:106-110).
// tiled: weights/scales in the quant.tile_fp4 / tile_fp4_scales layout (quant.py:118-134); rows % 16 == 0.
__global__ void __launch_bounds__(256) dequant_fp4_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ s,
                                                          long long rows, int K, int tiled, uint32_t* __restrict__ out) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;  // packed byte index in row-major order
    const int Kh = K >> 1;
    if (i >= rows * Kh) return;
    const long long n = i / Kh;
    const int j = (int)(i - n * Kh);
    const int ks = (2 * j) >> 5;
    long long wi, si;
    if (tiled) {
        const long long tile = (n >> 4) * (K >> 7) + (j >> 6);
        wi = tile * 1024 + (n & 15) * 64 + (j & 63);
        si = ((n >> 4) * (K >> 7) + (ks >> 2)) * 64 + (n & 15) * 4 + (ks & 3);
    } else {
        wi = i;
        si = n * (K >> 5) + ks;
    }
    const uint32_t byte = w[wi], sb = s[si];
    const uint32_t lo = f32_to_bf16_bits(__uint_as_float(e2m1_e8m0_f32_bits(byte & 15u, sb)));
    const uint32_t hi = f32_to_bf16_bits(__uint_as_float(e2m1_e8m0_f32_bits(byte >> 4, sb)));
    out[i] = lo | (hi << 16);
}

// ------------------------------------------------------------------------------------------ FP8 quant
// One 32-lane half-wave per 32-element group of a row. Input bf16 or fp32 with row stride ldx (elements);
// `permuted`: the row is in the 8-k permuted order of cukern.permute_x (within 8 k: 0,4,2,6,1,5,3,7, a
// bit reversal of k%8), codes/scales are written in natural k order. fq (optional) gets the fake-quantised
// values in the input's dtype and order (fused.fake_quant_fp8, fused.py:82-83).
__global__ void __launch_bounds__(256) quant_fp8_kernel(const void* __restrict__ x, int x_f32, long long rows, int K, long long ldx,
                                                        int permuted, uint8_t* __restrict__ codes, uint8_t* __restrict__ scales,
                                                        void* __restrict__ fq) {
    const long long gidx = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 5;  // group index
    const int lane = threadIdx.x & 31;
    const int gpr = K >> 5;
    if (gidx >= rows * gpr) return;
    const long long r = gidx / gpr;
    const int gk = (int)(gidx - r * gpr) * 32 + lane;  // position in the input row
    float v;
    if (x_f32) v = ((const float*)x)[r * ldx + gk];
    else v = bf16_to_f32(((const uint16_t*)x)[r * ldx + gk]);
    const float amax = wave_max32(fabsf(v));
    const int e = fq8_exponent(amax);
    const uint32_t code = fq8_code(v, e);
    const int nat = permuted ? ((gk & ~7) | ((gk & 1) << 2) | (gk & 2) | ((gk >> 2) & 1)) : gk;
    if (codes) codes[r * K + nat] = (uint8_t)code;
    if (scales && lane == 0) scales[r * gpr + (gk >> 5)] = (uint8_t)(e + 127);
    if (fq) {
        const float q = fq8_value(code, e);
        if (x_f32) ((float*)fq)[r * K + gk] = q;
        else ((uint16_t*)fq)[r * K + gk] = (uint16_t)f32_to_bf16_bits(q);
    }
}

// The same, 16 consecutive values per thread (two threads per 32-group): 16-byte loads and one 16-byte code
// store. Used when the pointers and strides allow 16-byte access and rows * K / 16 < 2^31.
__global__ void __launch_bounds__(256) quant_fp8_vec_kernel(const void* __restrict__ x, int x_f32, unsigned n_chunks, int K, long long ldx,
                                                            int permuted, uint8_t* __restrict__ codes, uint8_t* __restrict__ scales,
                                                            void* __restrict__ fq) {
    const unsigned t = blockIdx.x * 256u + threadIdx.x;   // 16-value chunk; a 32-group's two chunks are adjacent lanes
    if (t >= n_chunks) return;                            // n_chunks is even, so a lane pair is active together
    const unsigned cpr = (unsigned)K >> 4;
    const unsigned r = t / cpr, c = t - r * cpr;
    const int k0 = (int)c * 16;
    float f[16];
    if (x_f32) {
        const v4i* src = (const v4i*)((const float*)x + (long long)r * ldx + k0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const v4i w = src[j];
            f[4 * j] = __int_as_float(w.x); f[4 * j + 1] = __int_as_float(w.y);
            f[4 * j + 2] = __int_as_float(w.z); f[4 * j + 3] = __int_as_float(w.w);
        }
    } else {
        const v4i* src = (const v4i*)((const uint16_t*)x + (long long)r * ldx + k0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const v4i w = src[j];
            const uint32_t wd[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[8 * j + 2 * i] = bf16_to_f32(wd[i] & 0xFFFFu);
                f[8 * j + 2 * i + 1] = bf16_to_f32(wd[i] >> 16);
            }
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(f[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 2));
    const int e = fq8_exponent(amax);
    uint32_t q[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) q[i] = fq8_code(f[i], e);
    if (codes) {
        // natural position j holds input position (j & ~7) | bitrev3(j & 7) when the input is 8-k permuted
        uint32_t cw[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            cw[w] = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = 4 * w + b;
                const int src = permuted ? ((j & ~7) | ((j & 1) << 2) | (j & 2) | ((j >> 2) & 1)) : j;
                cw[w] |= q[src] << (8 * b);
            }
        }
        *(v4i*)(codes + (long long)r * K + k0) = v4i{(int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3]};
    }
    if (scales && (c & 1) == 0) scales[(long long)r * (K >> 5) + (c >> 1)] = (uint8_t)(e + 127);
    if (fq) {
        if (x_f32) {
            v4i* dst = (v4i*)((float*)fq + (long long)r * K + k0);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                dst[j] = v4i{__float_as_int(fq8_value(q[4 * j], e)), __float_as_int(fq8_value(q[4 * j + 1], e)),
                             __float_as_int(fq8_value(q[4 * j + 2], e)), __float_as_int(fq8_value(q[4 * j + 3], e))};
        } else {
            v4i* dst = (v4i*)((uint16_t*)fq + (long long)r * K + k0);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint32_t wd[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    wd[i] = f32_to_bf16_bits(fq8_value(q[8 * j + 2 * i], e)) | (f32_to_bf16_bits(fq8_value(q[8 * j + 2 * i + 1], e)) << 16);
                dst[j] = v4i{(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]};
            }
        }
    }
}

// ------------------------------------------------------------------------------------------ two-term FP8 split
// Activations that are not on the FP8 grid (any bf16 row, as the reference's bf16-operand GEMMs accept) as the sum of
// two E4M3 x E8M0 terms per 32-group (fp8_split16): hi = the per-32 FP8 rounding above (bit-identical codes and
// scales), lo = the residual rounded with a scale of its own. lo_flag (int32, optional; cleared by the entry first) is
// set when some lo code of any group is not zero, so kernels can skip the second term of FP8-grid input.
__global__ void __launch_bounds__(256) quant_fp8_split_kernel(const uint16_t* __restrict__ x, unsigned n_chunks, int K, long long ldx,
                                                              int permuted, uint8_t* __restrict__ hc, uint8_t* __restrict__ hs,
                                                              uint8_t* __restrict__ lc, uint8_t* __restrict__ ls, int* lo_flag) {
    const unsigned t = blockIdx.x * 256u + threadIdx.x;   // 16-value chunk; a 32-group's two chunks are adjacent lanes
    bool nz = false;
    if (t < n_chunks) {                                   // n_chunks is even, so a lane pair is active together
        const unsigned cpr = (unsigned)K >> 4;
        const unsigned r = t / cpr, c = t - r * cpr;
        const int k0 = (int)c * 16;
        const v4i* src = (const v4i*)(x + (long long)r * ldx + k0);
        v4i hi, lo;
        int e, e2;
        nz = fp8_split16(src[0], src[1], permuted, hi, lo, e, e2);
        *(v4i*)(hc + (long long)r * K + k0) = hi;
        *(v4i*)(lc + (long long)r * K + k0) = lo;
        if ((c & 1) == 0) {
            hs[(long long)r * (K >> 5) + (c >> 1)] = (uint8_t)(e + 127);
            ls[(long long)r * (K >> 5) + (c >> 1)] = (uint8_t)(e2 + 127);
        }
    }
    // one vector store of 1 per wave that saw a non-zero lo code (every writer stores the same value)
    const unsigned long long any = __ballot(nz);
    if (lo_flag && any && (threadIdx.x & 63) == (unsigned)__builtin_ctzll(any)) *(volatile int*)lo_flag = 1;
}

// inputs of at most this many 16-value chunks (262,144 values: 36 rows of 7168) take the 4-value-per-lane kernels
#define SMALL_CHUNKS 16384

// Small inputs (decode rows): the same split with 4 values per lane and a 32-group on 8 adjacent lanes. At one row of
// 7168 values the 16-value form runs 448 lanes through a serial chain of 16 encodings (two terms); this one runs 1792
// lanes through 4, which is what the launch's latency is made of at that size. Bit-identical to the 16-value form.
// permuted: the input holds 8-k permuted positions; lane pair (2m, 2m + 1) holds positions 8 m' .. 8 m' + 7 of one
// 8-block, and natural column j of the block sits at position (j & ~7) | bitrev3(j & 7), so each lane takes two of its
// values from the other lane of the pair.
__device__ __forceinline__ void unpermute_quad(float (&v)[4], bool odd) {
    // even lane: columns 0..3 = positions 0, 4, 2, 6 (own 0, pair 0, own 2, pair 2); odd lane: columns 4..7 =
    // positions 1, 5, 3, 7 (pair 1, own 1, pair 3, own 3)
    const float r0 = __shfl_xor(odd ? v[0] : v[1], 1), r1 = __shfl_xor(odd ? v[2] : v[3], 1);
    if (odd) {
        v[0] = r0;
        v[2] = r1;
    } else {
        v[1] = r0;
        v[3] = r1;
    }
}

__global__ void __launch_bounds__(256) quant_fp8_split_q4_kernel(const uint16_t* __restrict__ x, unsigned n_quads, int K, long long ldx,
                                                                 int permuted, uint8_t* __restrict__ hc, uint8_t* __restrict__ hs,
                                                                 uint8_t* __restrict__ lc, uint8_t* __restrict__ ls, int* lo_flag) {
    const unsigned t = blockIdx.x * 256u + threadIdx.x;   // 4-value quad; a 32-group's 8 quads are 8 aligned lanes
    bool nz = false;
    if (t < n_quads) {                                    // n_quads is a multiple of 8: a group's lanes are active together
        const unsigned qpr = (unsigned)K >> 2;
        const unsigned r = t / qpr, q = t - r * qpr;
        const int k0 = (int)q * 4;
        const uint2 w = *(const uint2*)(x + (long long)r * ldx + k0);
        float v[4] = {bf16_to_f32(w.x & 0xFFFFu), bf16_to_f32(w.x >> 16), bf16_to_f32(w.y & 0xFFFFu), bf16_to_f32(w.y >> 16)};
        if (permuted) unpermute_quad(v, (q & 1) != 0);
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
        const int e = fq8_exponent(amax);
        const uint32_t cw = fq8_code4_hw(v[0], v[1], v[2], v[3], e);
        float rr[4] = {__fsub_rn(v[0], fq8_value_hw<0>(cw, e)), __fsub_rn(v[1], fq8_value_hw<1>(cw, e)),   // the residuals, exact
                       __fsub_rn(v[2], fq8_value_hw<2>(cw, e)), __fsub_rn(v[3], fq8_value_hw<3>(cw, e))};
        float rmax = fmaxf(fmaxf(fabsf(rr[0]), fabsf(rr[1])), fmaxf(fabsf(rr[2]), fabsf(rr[3])));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 1, 8));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 2, 8));
        rmax = fmaxf(rmax, __shfl_xor(rmax, 4, 8));
        const int e2 = lo_exponent(rmax);
        const uint32_t cw2 = fq8_code4_hw(rr[0], rr[1], rr[2], rr[3], e2);
        nz = (cw2 & 0x7F7F7F7Fu) != 0;
        *(uint32_t*)(hc + (long long)r * K + k0) = cw;
        *(uint32_t*)(lc + (long long)r * K + k0) = cw2;
        if ((q & 7) == 0) {
            hs[(long long)r * (K >> 5) + (q >> 3)] = (uint8_t)(e + 127);
            ls[(long long)r * (K >> 5) + (q >> 3)] = (uint8_t)(e2 + 127);
        }
    }
    const unsigned long long any = __ballot(nz);
    if (lo_flag && any && (threadIdx.x & 63) == (unsigned)__builtin_ctzll(any)) *(volatile int*)lo_flag = 1;
}

__global__ void clear_flag_kernel(int* flag) {
    if (threadIdx.x == 0) *(volatile int*)flag = 0;
}

// ------------------------------------------------------------------------------------------ SwiGLU
// h = fq8(bf16(w * silu(min(g, L)) * clamp(u, +-L))) per 32 columns (fused.py:284-306; model.py:608-613).
// gu: fp32 or bf16 (gu_bf16) [rows, ld_gu] with gate in columns [0, I) and up in [I, 2I) (fused.swiglu_quant takes
// both: the routed path's fp32 GEMM output and the shared expert's bf16 linear output). Outputs: FP8 codes [rows, I] and E8M0
// [rows, I/32] (the down-projection operand), and optionally the bf16 values (fused.swiglu_quant's result,
// 8-k permuted when `permute`, fused.py:303-305).
__global__ void __launch_bounds__(256) swiglu_quant_kernel(const void* __restrict__ gu, int gu_bf16, long long ld_gu, const float* __restrict__ wt,
                                                           int rows, int inter, float limit, uint8_t* __restrict__ codes,
                                                           uint8_t* __restrict__ scales, uint16_t* __restrict__ hb, int permute) {
    const long long gidx = ((long long)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    const int lane = threadIdx.x & 31;
    const int gpr = inter >> 5;
    if (gidx >= (long long)rows * gpr) return;
    const int r = (int)(gidx / gpr);
    const int c = (int)(gidx - (long long)r * gpr) * 32 + lane;
    const long long ig = (long long)r * ld_gu + c, iu = ig + inter;
    float g = gu_bf16 ? bf16_to_f32(((const uint16_t*)gu)[ig]) : ((const float*)gu)[ig];
    float u = gu_bf16 ? bf16_to_f32(((const uint16_t*)gu)[iu]) : ((const float*)gu)[iu];
    if (limit > 0.f) {
        u = fminf(fmaxf(u, -limit), limit);
        g = fminf(g, limit);
    }
    float h = g * (1.0f / (1.0f + expf(-g))) * u;
    if (wt) h = h * wt[r];
    h = bf16_round(h);
    const float amax = wave_max32(fabsf(h));
    const int e = fq8_exponent(amax);
    const uint32_t code = fq8_code(h, e);
    if (codes) codes[(long long)r * inter + c] = (uint8_t)code;
    if (scales && lane == 0) scales[(long long)r * gpr + (c >> 5)] = (uint8_t)(e + 127);
    if (hb) {
        const int cc = permute ? ((c & ~7) | ((c & 1) << 2) | (c & 2) | ((c >> 2) & 1)) : c;
        hb[(long long)r * inter + cc] = (uint16_t)f32_to_bf16_bits(fq8_value(code, e));
    }
}

// The same per-element arithmetic, 16 columns per lane (a 32-column group is two adjacent lanes): 16-byte loads of gate
// and up, 16-byte stores of the codes and bf16 values. Needs 16-byte aligned rows and outputs.
__device__ __forceinline__ void load16_f(const void* p, int bf16, long long off, float* f) {
    if (!bf16) {
        const v4i* src = (const v4i*)((const float*)p + off);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const v4i w = src[j];
            f[4 * j] = __int_as_float(w.x); f[4 * j + 1] = __int_as_float(w.y);
            f[4 * j + 2] = __int_as_float(w.z); f[4 * j + 3] = __int_as_float(w.w);
        }
    } else {
        const v4i* src = (const v4i*)((const uint16_t*)p + off);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const v4i w = src[j];
            const uint32_t wd[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f[8 * j + 2 * i] = bf16_to_f32(wd[i] & 0xFFFFu);
                f[8 * j + 2 * i + 1] = bf16_to_f32(wd[i] >> 16);
            }
        }
    }
}

__global__ void __launch_bounds__(256) swiglu_quant_vec_kernel(const void* __restrict__ gu, int gu_bf16, long long ld_gu, const float* __restrict__ wt,
                                                               unsigned n_chunks, int inter, float limit, uint8_t* __restrict__ codes,
                                                               uint8_t* __restrict__ scales, uint16_t* __restrict__ hb, int permute) {
    const unsigned t = blockIdx.x * 256u + threadIdx.x;   // 16-column chunk; a 32-group's two chunks are adjacent lanes
    if (t >= n_chunks) return;                            // n_chunks is even, so a lane pair is active together
    const unsigned cpr = (unsigned)inter >> 4;
    const unsigned r = t / cpr, ch = t - r * cpr;
    const int c0 = (int)ch * 16;
    float g[16], u[16];
    load16_f(gu, gu_bf16, (long long)r * ld_gu + c0, g);
    load16_f(gu, gu_bf16, (long long)r * ld_gu + inter + c0, u);
    const float w = wt ? wt[r] : 1.f;
    float h[16];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float gg = g[i], uu = u[i];
        if (limit > 0.f) {
            uu = fminf(fmaxf(uu, -limit), limit);
            gg = fminf(gg, limit);
        }
        float v = gg * (1.0f / (1.0f + expf(-gg))) * uu;
        if (wt) v = v * w;
        v = bf16_round(v);
        h[i] = v;
        amax = fmaxf(amax, fabsf(v));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 2));
    const int e = fq8_exponent(amax);
    uint32_t q[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) q[i] = fq8_code(h[i], e);
    if (codes) {
        uint32_t cw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) cw[j] = q[4 * j] | (q[4 * j + 1] << 8) | (q[4 * j + 2] << 16) | (q[4 * j + 3] << 24);
        *(v4i*)(codes + (long long)r * inter + c0) = v4i{(int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3]};
    }
    if (scales && (ch & 1) == 0) scales[(long long)r * (inter >> 5) + (ch >> 1)] = (uint8_t)(e + 127);
    if (hb) {
        // permute: column j of the chunk is stored at (j & ~7) | bitrev3(j & 7), a map that is its own inverse, so
        // output position k holds column perm(k)
        v4i* dst = (v4i*)(hb + (long long)r * inter + c0);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t wd[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k0 = 8 * j + 2 * i, k1 = k0 + 1;
                const int s0 = permute ? ((k0 & ~7) | ((k0 & 1) << 2) | (k0 & 2) | ((k0 >> 2) & 1)) : k0;
                const int s1 = permute ? ((k1 & ~7) | ((k1 & 1) << 2) | (k1 & 2) | ((k1 >> 2) & 1)) : k1;
                wd[i] = f32_to_bf16_bits(fq8_value(q[s0], e)) | (f32_to_bf16_bits(fq8_value(q[s1], e)) << 16);
            }
            dst[j] = v4i{(int)wd[0], (int)wd[1], (int)wd[2], (int)wd[3]};
        }
    }
}

// Small inputs (decode rows): the same SwiGLU epilogue with 4 columns per lane and a 32-column group on 8 adjacent
// lanes (a serial chain of 4 exp / divide / encode steps per lane instead of 16). Bit-identical to the 16-column form.
// permute: the bf16 values go out 8-k permuted; the column <-> position map is its own inverse, so the lane pair
// exchanges values as unpermute_quad does.
__global__ void __launch_bounds__(256) swiglu_quant_q4_kernel(const void* __restrict__ gu, int gu_bf16, long long ld_gu, const float* __restrict__ wt,
                                                              unsigned n_quads, int inter, float limit, uint8_t* __restrict__ codes,
                                                              uint8_t* __restrict__ scales, uint16_t* __restrict__ hb, int permute) {
    const unsigned t = blockIdx.x * 256u + threadIdx.x;   // 4-column quad; a 32-group's 8 quads are 8 aligned lanes
    if (t >= n_quads) return;                             // n_quads is a multiple of 8: whole groups leave together
    const unsigned qpr = (unsigned)inter >> 2;
    const unsigned r = t / qpr, q = t - r * qpr;
    const int c0 = (int)q * 4;
    float g[4], u[4];
    const long long og = (long long)r * ld_gu + c0, ou = og + inter;
    if (!gu_bf16) {
        const v4f a = *(const v4f*)((const float*)gu + og), b = *(const v4f*)((const float*)gu + ou);
        g[0] = a.x; g[1] = a.y; g[2] = a.z; g[3] = a.w;
        u[0] = b.x; u[1] = b.y; u[2] = b.z; u[3] = b.w;
    } else {
        const uint2 a = *(const uint2*)((const uint16_t*)gu + og), b = *(const uint2*)((const uint16_t*)gu + ou);
        g[0] = bf16_to_f32(a.x & 0xFFFFu); g[1] = bf16_to_f32(a.x >> 16); g[2] = bf16_to_f32(a.y & 0xFFFFu); g[3] = bf16_to_f32(a.y >> 16);
        u[0] = bf16_to_f32(b.x & 0xFFFFu); u[1] = bf16_to_f32(b.x >> 16); u[2] = bf16_to_f32(b.y & 0xFFFFu); u[3] = bf16_to_f32(b.y >> 16);
    }
    const float w = wt ? wt[r] : 1.f;
    float h[4];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float gg = g[i], uu = u[i];
        if (limit > 0.f) {
            uu = fminf(fmaxf(uu, -limit), limit);
            gg = fminf(gg, limit);
        }
        float v = gg * (1.0f / (1.0f + expf(-gg))) * uu;
        if (wt) v = v * w;
        v = bf16_round(v);
        h[i] = v;
        amax = fmaxf(amax, fabsf(v));
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    const int e = fq8_exponent(amax);
    const uint32_t qw = fq8_code4_hw(h[0], h[1], h[2], h[3], e);
    if (codes) *(uint32_t*)(codes + (long long)r * inter + c0) = qw;
    if (scales && (q & 7) == 0) scales[(long long)r * (inter >> 5) + (q >> 3)] = (uint8_t)(e + 127);
    if (hb) {
        float o[4] = {fq8_value_hw<0>(qw, e), fq8_value_hw<1>(qw, e), fq8_value_hw<2>(qw, e), fq8_value_hw<3>(qw, e)};
        if (permute) unpermute_quad(o, (q & 1) != 0);
        *(uint2*)(hb + (long long)r * inter + c0) = uint2{f32_to_bf16_bits(o[0]) | (f32_to_bf16_bits(o[1]) << 16),
                                                          f32_to_bf16_bits(o[2]) | (f32_to_bf16_bits(o[3]) << 16)};
    }
}

// ------------------------------------------------------------------------------------------ C ABI
extern "C" int dsv41_dequant_fp4(const uint8_t* w, const uint8_t* s, long long rows, int K, int tiled, uint16_t* out, void* stream) {
    if (!w || !s || !out || rows < 0 || K <= 0 || (K & 31) || (tiled && ((rows & 15) || (K & 127)))) return DSV41_EINVAL;
    const long long n = rows * (K / 2);
    if (n == 0) return 0;
    dequant_fp4_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(w, s, rows, K, tiled, (uint32_t*)out);
    return (int)hipGetLastError();
}

extern "C" int dsv41_quant_fp8(const void* x, int x_f32, long long rows, int K, long long ldx, int permuted,
                               uint8_t* codes, uint8_t* scales, void* fq, void* stream) {
    if (!x || rows < 0 || K <= 0 || (K & 31) || ldx < K || (!codes && !scales && !fq)) return DSV41_EINVAL;
    const long long groups = rows * (K / 32);
    if (groups == 0) return 0;
    const int esz = x_f32 ? 4 : 2;
    const bool vec = groups * 2 < (1ll << 31) && ((ldx * esz) & 15) == 0 && (((uintptr_t)x) & 15) == 0 && (((uintptr_t)codes) & 15) == 0 &&
                     (((uintptr_t)fq) & 15) == 0 && (K & 15) == 0;
    if (vec) {
        const unsigned n_chunks = (unsigned)(groups * 2);
        quant_fp8_vec_kernel<<<(n_chunks + 255) / 256, 256, 0, (hipStream_t)stream>>>(x, x_f32, n_chunks, K, ldx, permuted, codes, scales, fq);
    } else {
        quant_fp8_kernel<<<(unsigned)((groups * 32 + 255) / 256), 256, 0, (hipStream_t)stream>>>(x, x_f32, rows, K, ldx, permuted, codes, scales, fq);
    }
    return (int)hipGetLastError();
}

extern "C" int dsv41_quant_fp8_split(const uint16_t* x, long long rows, int K, long long ldx, int permuted, uint8_t* hc, uint8_t* hs,
                                     uint8_t* lc, uint8_t* ls, int* lo_flag, void* stream) {
    if (!x || !hc || !hs || !lc || !ls || rows < 0 || K <= 0 || (K & 31) || ldx < K || (ldx & 7) || (((uintptr_t)x) & 15) ||
        (((uintptr_t)hc) & 15) || (((uintptr_t)lc) & 15))
        return DSV41_EINVAL;
    const long long n = rows * (K / 16);
    if (n >= (1ll << 31)) return DSV41_EINVAL;
    hipStream_t st = (hipStream_t)stream;
    if (lo_flag) clear_flag_kernel<<<1, 64, 0, st>>>(lo_flag);
    if (n > 0 && n <= SMALL_CHUNKS) {   // decode rows: 4 values per lane
        const unsigned nq = (unsigned)(4 * n);
        quant_fp8_split_q4_kernel<<<(nq + 255) / 256, 256, 0, st>>>(x, nq, K, ldx, permuted, hc, hs, lc, ls, lo_flag);
    } else if (n > 0) {
        quant_fp8_split_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(x, (unsigned)n, K, ldx, permuted, hc, hs, lc, ls, lo_flag);
    }
    return (int)hipGetLastError();
}

extern "C" int dsv41_swiglu_quant(const void* gu, int gu_bf16, long long ld_gu, const float* wt, int rows, int inter, float limit,
                                  uint8_t* codes, uint8_t* scales, uint16_t* h_bf16, int permute, void* stream) {
    if (!gu || rows < 0 || inter <= 0 || (inter & 31) || ld_gu < 2LL * inter || (!codes && !scales && !h_bf16)) return DSV41_EINVAL;
    const long long groups = (long long)rows * (inter / 32);
    if (groups == 0) return 0;
    const int esz = gu_bf16 ? 2 : 4;
    if (groups * 2 <= SMALL_CHUNKS && (((uintptr_t)gu) & 15) == 0 && (ld_gu & 3) == 0 && (((uintptr_t)codes) & 3) == 0 &&
        (((uintptr_t)h_bf16) & 7) == 0) {   // decode rows: 4 columns per lane
        const unsigned nq = (unsigned)(groups * 8);
        swiglu_quant_q4_kernel<<<(nq + 255) / 256, 256, 0, (hipStream_t)stream>>>(gu, gu_bf16, ld_gu, wt, nq, inter, limit, codes, scales,
                                                                                  h_bf16, permute);
        return (int)hipGetLastError();
    }
    const bool vec = groups * 2 < (1ll << 31) && (((uintptr_t)gu) & 15) == 0 && ((ld_gu * esz) & 15) == 0 && (((uintptr_t)codes) & 15) == 0 &&
                     (((uintptr_t)h_bf16) & 15) == 0;
    if (vec) {
        const unsigned n_chunks = (unsigned)(groups * 2);
        swiglu_quant_vec_kernel<<<(n_chunks + 255) / 256, 256, 0, (hipStream_t)stream>>>(gu, gu_bf16, ld_gu, wt, n_chunks, inter, limit, codes,
                                                                                          scales, h_bf16, permute);
        return (int)hipGetLastError();
    }
    swiglu_quant_kernel<<<(unsigned)((groups * 32 + 255) / 256), 256, 0, (hipStream_t)stream>>>(gu, gu_bf16, ld_gu, wt, rows, inter, limit, codes, scales, h_bf16, permute);
    return (int)hipGetLastError();
}
