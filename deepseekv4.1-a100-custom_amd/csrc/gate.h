// The MoE gate of one token row, computed by one wave (fused2.gate_topk, fused2.py:418-452; model.MoE.gate,
// model.py:391-404): scoring function, + bias for the selection only, top-k with the lowest index winning ties,
// weights renormalised (+1e-20) and scaled. Lane l owns scores e = l, l + 64, ... in registers; every reduction
// is a DPP row operation (no LDS round trips); each of the topk rounds is one 64-bit max-reduction over keys
// (order(score + bias) << 32 | ~index). On return lane k < topk holds the k-th expert id and its weight.
#pragma once
#include "common.h"

template <int PER>
__device__ __forceinline__ void gate_row_wave(const float* __restrict__ S, const float* __restrict__ bias, int E, float temp, int topk,
                                              float route_scale, int mode, int norm, int* out_i, float* out_w) {
    const int lane = threadIdx.x & 63;
    float s[PER];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = lane + 64 * i;
        s[i] = e < E ? S[e] / temp : -INFINITY;
        mx = fmaxf(mx, s[i]);
    }
    // scoring function (mode 0 sqrt(softplus), 1 sigmoid, 2 softmax), fused2.py:433-440
    if (mode == 2) {
        mx = wave_reduce_max(mx);
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            s[i] = lane + 64 * i < E ? expf(s[i] - mx) : 0.f;
            sum += s[i];
        }
        sum = wave_reduce_sum(sum);
#pragma unroll
        for (int i = 0; i < PER; ++i) s[i] = s[i] / sum;
    } else {
#pragma unroll
        for (int i = 0; i < PER; ++i)
            s[i] = mode == 1 ? 1.0f / (1.0f + expf(-s[i])) : sqrtf(s[i] > 20.f ? s[i] : log1pf(expf(s[i])));
    }
    unsigned long long key[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int e = lane + 64 * i;
        const float v = e < E ? s[i] + (bias ? bias[e] : 0.f) : -INFINITY;
        // invalid entries and NaN scores get key 0: they never beat a real candidate
        key[i] = (e < E && v == v) ? ((unsigned long long)float_order_key(v) << 32) | (unsigned)(0xFFFFFFFFu - (unsigned)e) : 0ull;
    }
    float wsum = 0.f, my_w = 0.f;
    int my_i = 0;
    for (int k = 0; k < topk; ++k) {
        unsigned long long best = 0;
#pragma unroll
        for (int i = 0; i < PER; ++i) best = key[i] > best ? key[i] : best;
        best = wave_reduce_max_u64(best);
        // no candidate left (every remaining score NaN): emit index k, so no index is ever >= E
        const int bi = best ? (int)(0xFFFFFFFFu - (unsigned)best) : k;
        const int owner = bi & 63, slot = bi >> 6;
        float w = 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i)
            if (i == slot && lane == owner) { w = s[i]; key[i] = 0; }
        w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), owner));
        wsum += w;
        if (lane == k) { my_w = w; my_i = bi; }
    }
    *out_i = my_i;
    *out_w = norm ? my_w / (wsum + 1e-20f) * route_scale : my_w * route_scale;
}
