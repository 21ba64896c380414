// The MoE gate of one token row, computed by one wave (fused2.gate_topk, fused2.py:418-452; model.MoE.gate,
// model.py:391-404): scoring function, + bias for the selection only, top-k with the lowest index winning ties,
// weights renormalised (+1e-20) and scaled. Lane l owns the contiguous scores e = l * PER .. l * PER + PER - 1
// in registers, so a lower lane always holds lower indices: each of the topk rounds is one 32-bit DPP
// max-reduction over the lanes' current maxima (order-preserving keys of score + bias) and one ballot, whose
// lowest set lane is the winner (ties -> lowest index). Only the winning lane rescans its PER keys. On return
// lane k < topk holds the k-th expert id and its weight.
#pragma once
#include "common.h"

// The gate's state in one wave. prepare(): the scores and selection keys of the row; pick(k): the k-th selection
// round (the same result in every lane). A caller can act on each expert as soon as its round is done.
template <int PER>
struct GateRow {
    float s[PER];
    unsigned key[PER];
    unsigned lk;   // the lane's best remaining key, its slot (lowest on ties) and score
    int li;
    float ls;
    // the logits may arrive as nparts partial sums (a split-K router GEMV); loads go out Q parts at a time
    static constexpr int Q = PER <= 8 ? 8 : 1;
    float raw[Q][PER];   // the first batch of parts, loaded ahead of prepare() by load_logits()
    bool loaded = false;

    // issue the loads of the first Q parts of logits now (a caller can do this first thing, before any barrier).
    // Addresses are clamped (to the last entry, the last part), so no branch splits the batch; prepare() masks.
    __device__ __forceinline__ void load_logits(const float* __restrict__ S, int E, int nparts, long long pstride) {
        const int e0 = (threadIdx.x & 63) * PER;
#pragma unroll
        for (int q = 0; q < (nparts == 1 ? 1 : Q); ++q) {
            const long long off = (long long)min(q, nparts - 1) * pstride;
#pragma unroll
            for (int i = 0; i < PER; ++i) raw[q][i] = S[off + min(e0 + i, E - 1)];
        }
        loaded = true;
    }

    __device__ __forceinline__ void rescan() {   // selects, not branches: no exec-mask changes per slot
        lk = 0u;
        li = 0;
        ls = 0.f;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const bool gt = key[i] > lk;
            lk = gt ? key[i] : lk;
            li = gt ? i : li;
            ls = gt ? s[i] : ls;
        }
    }

    __device__ __forceinline__ void prepare(const float* __restrict__ S, int nparts, long long pstride, const float* __restrict__ bias, int E,
                                            float temp, int mode) {
        const int lane = threadIdx.x & 63;
        const int e0 = lane * PER;
        float mx = -INFINITY;
        // partial sums are added in ascending part order; one part (plain logits) is a single batch of PER loads
        float v[PER];
#pragma unroll
        for (int i = 0; i < PER; ++i) v[i] = 0.f;
        if (nparts == 1) {
#pragma unroll
            for (int i = 0; i < PER; ++i) v[i] = e0 + i < E ? (loaded ? raw[0][i] : S[e0 + i]) : 0.f;
        }
        for (int p0 = 0; nparts > 1 && p0 < nparts; p0 += Q) {
            float t[Q][PER];
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const long long off = (long long)min(p0 + q, nparts - 1) * pstride;
#pragma unroll
                for (int i = 0; i < PER; ++i) t[q][i] = e0 + i < E ? (loaded && p0 == 0 ? raw[q][i] : S[off + e0 + i]) : 0.f;
            }
#pragma unroll
            for (int q = 0; q < Q; ++q)
                if (p0 + q < nparts)
#pragma unroll
                    for (int i = 0; i < PER; ++i) v[i] += t[q][i];
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            s[i] = e0 + i < E ? (temp == 1.0f ? v[i] : v[i] / temp) : -INFINITY;   // x / 1 == x exactly
            mx = fmaxf(mx, s[i]);
        }
        // scoring function (mode 0 sqrt(softplus), 1 sigmoid, 2 softmax), fused2.py:433-440
        if (mode == 2) {
            mx = wave_reduce_max(mx);
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                s[i] = e0 + i < E ? expf(s[i] - mx) : 0.f;
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
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const float b = e0 + i < E ? s[i] + (bias ? bias[e0 + i] : 0.f) : -INFINITY;
            // invalid entries and NaN scores get key 0: every real candidate's key is larger
            key[i] = (e0 + i < E && b == b) ? float_order_key(b) : 0u;
        }
        rescan();
    }

    // round k: the id (k when no candidate is left, every remaining score NaN, so no id is ever >= E) and score.
    // Branch-free: the winner's key is cleared through a per-lane bit mask and every lane rescans (only the
    // owner's keys changed), so no scalar branch tree is built on the winning slot.
    __device__ __forceinline__ void pick(int k, int* id, float* w) {
        const int lane = threadIdx.x & 63;
        const unsigned best = wave_reduce_max_u32z(lk);
        const unsigned long long m = __ballot(best != 0u && lk == best);
        const int owner = m ? (int)__builtin_ctzll(m) : 0;
        const int slot = __builtin_amdgcn_readlane(li, owner);
        *id = m ? owner * PER + slot : k;
        *w = m ? __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ls), owner)) : 0.f;
        const unsigned clear = (m && lane == owner) ? 1u << li : 0u;
#pragma unroll
        for (int i = 0; i < PER; ++i) key[i] = ((clear >> i) & 1u) ? 0u : key[i];
        rescan();
    }
};

// the routing weight of a pick: renormalised over the topk picks (+1e-20) and scaled, fused2.py:445-450
__device__ __forceinline__ float gate_weight(float w, float wsum, float route_scale, int norm) {
    return norm ? w / (wsum + 1e-20f) * route_scale : w * route_scale;
}

template <int PER>
__device__ __forceinline__ void gate_row_wave(const float* __restrict__ S, int nparts, long long pstride, const float* __restrict__ bias, int E,
                                              float temp, int topk, float route_scale, int mode, int norm, int* out_i, float* out_w) {
    const int lane = threadIdx.x & 63;
    GateRow<PER> gr;
    gr.prepare(S, nparts, pstride, bias, E, temp, mode);
    float wsum = 0.f, my_w = 0.f;
    int my_i = 0;
    for (int k = 0; k < topk; ++k) {
        int id;
        float w;
        gr.pick(k, &id, &w);
        wsum += w;
        if (lane == k) { my_w = w; my_i = id; }
    }
    *out_i = my_i;
    *out_w = gate_weight(my_w, wsum, route_scale, norm);
}
