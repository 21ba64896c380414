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

// ------------------------------------------------------------------------------------------ hyper-connections
// The decode block's steps either side of the experts when the residual is kept as hc = 4 streams (fused2.py:189-236,
// 474-538):
//   hc_pre_norm_quant: a  = bf16(sum_h pre[h] * x[h])              (the hyper-connection pre-mix, h ascending)
//                      y  = bf16(a * (1 / sqrt(mean(a^2) + eps)) * w)  (rmsnorm, fp32 statistics)
//                      yq = fake_quant_fp8(y) per 32; optional y as fp32 and yq in the 8-k permuted order
//   hc_post:           x  = bf16(sum_k y2[k] + ys) (the MoE pair rows and the shared expert; or a given x)
//                      r[i] <- bf16(post[i] * x + sum_j comb[j][i] * r[j])  for the 4 streams, in place
// One workgroup per row for the pre step (each thread 8 consecutive elements); the post step takes 4 columns per
// thread.
#define HC_MAX 4

__global__ void __launch_bounds__(NORM_THREADS) hc_pre_norm_quant_kernel(const uint16_t* __restrict__ x, long long ldx, int hc,
                                                                         const float* __restrict__ pre, long long ldp,
                                                                         const uint16_t* __restrict__ w, float eps, int D,
                                                                         uint16_t* __restrict__ y, long long ldy, uint16_t* __restrict__ yq,
                                                                         long long ldq, float* __restrict__ yf, long long ldf,
                                                                         uint16_t* __restrict__ yqp, long long ldqp) {
    __shared__ float s_part[NORM_THREADS / 64];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool mine = tid < (D >> 3);
    float p[HC_MAX];
#pragma unroll
    for (int h = 0; h < HC_MAX; ++h) p[h] = h < hc ? pre[(long long)b * ldp + h] : 0.f;
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) a[j] = 0.f;
    float ss = 0.f;
    if (mine) {
#pragma unroll
        for (int h = 0; h < HC_MAX; ++h) {
            if (h >= hc) break;
            const v4i xv = *(const v4i*)(x + (long long)b * ldx + (long long)h * D + tid * 8);
            const uint32_t xw[4] = {(uint32_t)xv.x, (uint32_t)xv.y, (uint32_t)xv.z, (uint32_t)xv.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                a[2 * j] = fmaf(p[h], bf16_to_f32(xw[j] & 0xFFFFu), a[2 * j]);
                a[2 * j + 1] = fmaf(p[h], bf16_to_f32(xw[j] >> 16), a[2 * j + 1]);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            a[j] = bf16_round(a[j]);   // the pre-mix output is a bf16 tensor
            ss += a[j] * a[j];
        }
    }
    ss = wave_reduce_sum(ss);
    if (lane == 0) s_part[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int i = 0; i < NORM_THREADS / 64; ++i) tot += s_part[i];
    const float inv = 1.0f / sqrtf(tot / (float)D + eps);
    if (!mine) return;
    const v4i ww = *(const v4i*)(w + tid * 8);
    const uint32_t wv4[4] = {(uint32_t)ww.x, (uint32_t)ww.y, (uint32_t)ww.z, (uint32_t)ww.w};
    float v[8];
    uint32_t nw[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        v[2 * j] = bf16_round(a[2 * j] * inv * bf16_to_f32(wv4[j] & 0xFFFFu));
        v[2 * j + 1] = bf16_round(a[2 * j + 1] * inv * bf16_to_f32(wv4[j] >> 16));
        nw[j] = f32_to_bf16_bits(v[2 * j]) | (f32_to_bf16_bits(v[2 * j + 1]) << 16);
    }
    *(v4i*)(y + (long long)b * ldy + tid * 8) = v4i{(int)nw[0], (int)nw[1], (int)nw[2], (int)nw[3]};
    if (yf) {
        *(v4f*)(yf + (long long)b * ldf + tid * 8) = v4f{v[0], v[1], v[2], v[3]};
        *(v4f*)(yf + (long long)b * ldf + tid * 8 + 4) = v4f{v[4], v[5], v[6], v[7]};
    }
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 4));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 4));
    const int e = fq8_exponent(amax);
    uint32_t q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = f32_to_bf16_bits(fq8_value(fq8_code(v[j], e), e));
    if (yq) {
        const uint32_t qw[4] = {q[0] | (q[1] << 16), q[2] | (q[3] << 16), q[4] | (q[5] << 16), q[6] | (q[7] << 16)};
        *(v4i*)(yq + (long long)b * ldq + tid * 8) = v4i{(int)qw[0], (int)qw[1], (int)qw[2], (int)qw[3]};
    }
    if (yqp) {
        // the 8-k permuted order (0, 4, 2, 6, 1, 5, 3, 7 within each 8, cukern.permute_x / fused2._perm8): slot s holds
        // element perm[s]
        const uint32_t pw[4] = {q[0] | (q[4] << 16), q[2] | (q[6] << 16), q[1] | (q[5] << 16), q[3] | (q[7] << 16)};
        *(v4i*)(yqp + (long long)b * ldqp + tid * 8) = v4i{(int)pw[0], (int)pw[1], (int)pw[2], (int)pw[3]};
    }
}

__global__ void __launch_bounds__(256) hc_post_kernel(const uint16_t* __restrict__ x, long long ldx, const float* __restrict__ y2,
                                                      long long y2_row, long long y2_sum, int nsum, const uint16_t* __restrict__ ys,
                                                      long long ldys, uint16_t* __restrict__ res, long long ldr, const float* __restrict__ post,
                                                      long long ldpost, const float* __restrict__ comb, long long ldcomb, int D) {
    const int b = blockIdx.y;
    const int n = (blockIdx.x * blockDim.x + threadIdx.x) * 4;
    if (n >= D) return;
    float xv[4];
    if (nsum > 0) {
        const float* src = y2 + (long long)b * y2_row + n;
        v4f s = *(const v4f*)src;
        for (int k = 1; k < nsum; ++k) s += *(const v4f*)(src + (long long)k * y2_sum);
        xv[0] = s.x; xv[1] = s.y; xv[2] = s.z; xv[3] = s.w;
        if (ys) {
            const uint2 yv = *(const uint2*)(ys + (long long)b * ldys + n);
            xv[0] += bf16_to_f32(yv.x & 0xFFFFu); xv[1] += bf16_to_f32(yv.x >> 16);
            xv[2] += bf16_to_f32(yv.y & 0xFFFFu); xv[3] += bf16_to_f32(yv.y >> 16);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[j] = bf16_round(xv[j]);
    } else {
        const uint2 v = *(const uint2*)(x + (long long)b * ldx + n);
        xv[0] = bf16_to_f32(v.x & 0xFFFFu); xv[1] = bf16_to_f32(v.x >> 16);
        xv[2] = bf16_to_f32(v.y & 0xFFFFu); xv[3] = bf16_to_f32(v.y >> 16);
    }
    uint16_t* r = res + (long long)b * ldr + n;
    float rv[HC_MAX][4];
#pragma unroll
    for (int j = 0; j < HC_MAX; ++j) {
        const uint2 v = *(const uint2*)(r + (long long)j * D);
        rv[j][0] = bf16_to_f32(v.x & 0xFFFFu); rv[j][1] = bf16_to_f32(v.x >> 16);
        rv[j][2] = bf16_to_f32(v.y & 0xFFFFu); rv[j][3] = bf16_to_f32(v.y >> 16);
    }
    const float* pb = post + (long long)b * ldpost;
    const float* cb = comb + (long long)b * ldcomb;
#pragma unroll
    for (int i = 0; i < HC_MAX; ++i) {
        uint32_t o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float acc = pb[i] * xv[c];
#pragma unroll
            for (int j = 0; j < HC_MAX; ++j) acc = fmaf(cb[j * HC_MAX + i], rv[j][c], acc);
            o[c] = f32_to_bf16_bits(acc);
        }
        *(uint2*)(r + (long long)i * D) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
    }
}

extern "C" int dsv41_hc_pre_norm_quant(const uint16_t* x, long long ldx, int hc, const float* pre, long long ldp, const uint16_t* w, float eps,
                                       int B, int D, uint16_t* y, long long ldy, uint16_t* yq, long long ldq, float* yf, long long ldf,
                                       uint16_t* yqp, long long ldqp, void* stream) {
    if (!x || !pre || !w || !y || B < 1 || hc < 1 || hc > HC_MAX || D <= 0 || (D & 31) || D / 8 > NORM_THREADS || ldx < (long long)hc * D ||
        ldy < D || (yq && ldq < D) || (yf && ldf < D) || (yqp && ldqp < D) || ((ldx | ldy | D | (yq ? ldq : 0) | (yqp ? ldqp : 0)) & 7) ||
        (yf && (ldf & 3)) || !(eps >= 0.f) ||
        ((((uintptr_t)x) | ((uintptr_t)w) | ((uintptr_t)y) | ((uintptr_t)yq) | ((uintptr_t)yf) | ((uintptr_t)yqp)) & 15))
        return DSV41_EINVAL;
    hc_pre_norm_quant_kernel<<<B, NORM_THREADS, 0, (hipStream_t)stream>>>(x, ldx, hc, pre, ldp, w, eps, D, y, ldy, yq, ldq, yf, ldf, yqp, ldqp);
    return (int)hipGetLastError();
}

extern "C" int dsv41_hc_post(const uint16_t* x, long long ldx, const float* y2, long long y2_row, long long y2_sum, int nsum, const uint16_t* ys,
                             long long ldys, uint16_t* res, long long ldr, const float* post, long long ldpost, const float* comb, long long ldcomb,
                             int B, int D, void* stream) {
    if (!res || !post || !comb || B < 1 || D <= 0 || (D & 3) || nsum < 0 || (nsum == 0 && !x) || (nsum > 0 && !y2) || ldr < (long long)HC_MAX * D ||
        ((((uintptr_t)res) | ((uintptr_t)x) | ((uintptr_t)ys)) & 7) || (((uintptr_t)y2) & 15) || ((ldr | (x ? ldx : 0) | (ys ? ldys : 0)) & 3) ||
        (nsum > 0 && ((y2_row | y2_sum) & 3)))
        return DSV41_EINVAL;
    const dim3 grid((unsigned)((D / 4 + 255) / 256), (unsigned)B);
    hc_post_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(x, ldx, y2, y2_row, y2_sum, nsum, ys, ldys, res, ldr, post, ldpost, comb, ldcomb, D);
    return (int)hipGetLastError();
}
