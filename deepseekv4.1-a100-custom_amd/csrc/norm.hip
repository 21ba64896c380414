// Residual + RMSNorm + FP8 fake-quantisation of token rows: the step that joins two MoE layers in the decode
// stack. For row t:
//   r      = bf16(x[t] + y[t])                             (the bf16 residual stream; x, y bf16)
//   xn     = bf16(r * rsqrt(mean(r^2) + eps) * (w ? w : 1)) (fused.rmsnorm, fused.py:92-110, fp32 statistics)
//   xq     = fake_quant_fp8(xn) per 32 along H              (quant.py:34-54)
// Outputs: xn (the next layer's router input, model.py:391 routes on the unquantised activations) and xq (its
// experts' input). One workgroup per row; each thread owns 8 consecutive elements (one 16-byte load per input),
// four threads one FP8 group.
#include "common.h"

#define NORM_THREADS 1024

__global__ void __launch_bounds__(NORM_THREADS) residual_rmsnorm_quant_kernel(const uint16_t* __restrict__ x, long long ldx,
                                                                               const uint16_t* __restrict__ y, long long ldy,
                                                                               const uint16_t* __restrict__ w, float eps, int H,
                                                                               uint16_t* __restrict__ xn, long long ldn,
                                                                               uint16_t* __restrict__ xq, long long ldq) {
    __shared__ float s_part[NORM_THREADS / 64];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nvec = H >> 3;
    float r[8];
    float ss = 0.f;
    const bool mine = tid < nvec;
    if (mine) {
        const v4i xv = *(const v4i*)(x + (long long)t * ldx + tid * 8);
        const v4i yv = *(const v4i*)(y + (long long)t * ldy + tid * 8);
        const uint32_t xw[4] = {(uint32_t)xv.x, (uint32_t)xv.y, (uint32_t)xv.z, (uint32_t)xv.w};
        const uint32_t yw[4] = {(uint32_t)yv.x, (uint32_t)yv.y, (uint32_t)yv.z, (uint32_t)yv.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r[2 * j] = bf16_round(bf16_to_f32(xw[j] & 0xFFFFu) + bf16_to_f32(yw[j] & 0xFFFFu));
            r[2 * j + 1] = bf16_round(bf16_to_f32(xw[j] >> 16) + bf16_to_f32(yw[j] >> 16));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += r[j] * r[j];
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = 0.f;
    }
    // sum of squares: DPP within the wave, then the waves' partials in a fixed order
    ss = wave_reduce_sum(ss);
    if (lane == 0) s_part[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < NORM_THREADS / 64; ++i) tot += s_part[i];
    const float inv = 1.0f / sqrtf(tot / (float)H + eps);
    if (!mine) return;
    float v[8];
    uint32_t nw[4];
    uint32_t wv4[4] = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};   // bf16 1.0 pairs
    if (w) {
        const v4i ww = *(const v4i*)(w + tid * 8);
        wv4[0] = (uint32_t)ww.x; wv4[1] = (uint32_t)ww.y; wv4[2] = (uint32_t)ww.z; wv4[3] = (uint32_t)ww.w;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float a = bf16_round(r[2 * j] * inv * bf16_to_f32(wv4[j] & 0xFFFFu));
        const float b = bf16_round(r[2 * j + 1] * inv * bf16_to_f32(wv4[j] >> 16));
        v[2 * j] = a;
        v[2 * j + 1] = b;
        nw[j] = f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
    }
    *(v4i*)(xn + (long long)t * ldn + tid * 8) = v4i{(int)nw[0], (int)nw[1], (int)nw[2], (int)nw[3]};
    // per-32 FP8 fake quantisation: the 4 threads of a group exchange their amax (a quad is always active together)
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 4));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 4));
    const int e = fq8_exponent(amax);
    uint32_t qw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        qw[j] = f32_to_bf16_bits(fq8_value(fq8_code(v[2 * j], e), e)) | (f32_to_bf16_bits(fq8_value(fq8_code(v[2 * j + 1], e), e)) << 16);
    *(v4i*)(xq + (long long)t * ldq + tid * 8) = v4i{(int)qw[0], (int)qw[1], (int)qw[2], (int)qw[3]};
}

extern "C" int dsv41_residual_rmsnorm_quant(const uint16_t* x, long long ldx, const uint16_t* y, long long ldy, const uint16_t* w, float eps,
                                            int M, int H, uint16_t* xn, long long ldn, uint16_t* xq, long long ldq, void* stream) {
    if (!x || !y || !xn || !xq || M < 1 || H <= 0 || (H & 31) || H / 8 > NORM_THREADS || ldx < H || ldy < H || ldn < H || ldq < H ||
        ((ldx | ldy | ldn | ldq) & 7) || ((((uintptr_t)x) | ((uintptr_t)y) | ((uintptr_t)xn) | ((uintptr_t)xq) | ((uintptr_t)w)) & 15) ||
        !(eps >= 0.f))
        return DSV41_EINVAL;
    residual_rmsnorm_quant_kernel<<<M, NORM_THREADS, 0, (hipStream_t)stream>>>(x, ldx, y, ldy, w, eps, H, xn, ldn, xq, ldq);
    return (int)hipGetLastError();
}
