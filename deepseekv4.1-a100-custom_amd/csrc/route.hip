// Routing kernels: the MoE gate (fused2.gate_topk, fused2.py:418-471; model.MoE.gate, model.py:391-404) and the
// expert bucketing of (token, expert) pairs (cukern.moe_dispatch -> p2p.cu:90-132).
//
// gate_topk_kernel: one workgroup per token row. Scores -> softmax / sigmoid / sqrt(softplus), + bias for the
// selection only, TOPK rounds of a block-wide arg-max (lowest index wins ties, fused2.py:441), weights
// renormalised (+1e-20) and scaled.
// moe_dispatch_kernel: one workgroup, any number of pairs. Histogram (LDS atomics), exclusive scan over experts,
// then a STABLE scatter: pairs keep ascending pair order within an expert (the reference's order is arbitrary,
// p2p.cu:91-93; a stable order makes the tables reproducible). Rounds of blockDim pairs; within a wave the rank
// among same-expert lanes comes from ballots, across waves from per-wave counts in LDS.
#include "common.h"

#define GATE_THREADS 256
#define GATE_MAX_E 2048

__device__ __forceinline__ void argmax_pair(float& v, int& i, float v2, int i2) {
    if (v2 > v || (v2 == v && i2 < i)) { v = v2; i = i2; }
}

__global__ void __launch_bounds__(GATE_THREADS) gate_topk_kernel(const float* __restrict__ scores, long long lds, const float* __restrict__ bias,
                                                                 int E, float temp, int topk, float route_scale, int mode, int norm,
                                                                 int* __restrict__ eid, float* __restrict__ wt) {
    __shared__ float s_s[GATE_MAX_E], s_b[GATE_MAX_E];
    __shared__ float s_rv[GATE_THREADS / WAVE];
    __shared__ int s_ri[GATE_THREADS / WAVE];
    __shared__ float s_w[32];
    __shared__ int s_i[32];
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* S = scores + (long long)row * lds;
    // scoring function (mode 0 sqrt(softplus), 1 sigmoid, 2 softmax), fused2.py:433-440
    float lmax = -INFINITY;
    for (int e = tid; e < E; e += GATE_THREADS) {
        const float s = S[e] / temp;
        s_s[e] = s;
        lmax = fmaxf(lmax, s);
    }
    __syncthreads();
    if (mode == 2) {
        for (int o = 32; o > 0; o >>= 1) lmax = fmaxf(lmax, __shfl_xor(lmax, o));
        if (lane == 0) s_rv[wave] = lmax;
        __syncthreads();
        float mx = s_rv[0];
        for (int w = 1; w < GATE_THREADS / WAVE; ++w) mx = fmaxf(mx, s_rv[w]);
        __syncthreads();
        float lsum = 0.f;
        for (int e = tid; e < E; e += GATE_THREADS) {
            const float ex = expf(s_s[e] - mx);
            s_s[e] = ex;
            lsum += ex;
        }
        for (int o = 32; o > 0; o >>= 1) lsum += __shfl_xor(lsum, o);
        if (lane == 0) s_rv[wave] = lsum;
        __syncthreads();
        float tot = 0.f;
        for (int w = 0; w < GATE_THREADS / WAVE; ++w) tot += s_rv[w];
        for (int e = tid; e < E; e += GATE_THREADS) s_s[e] = s_s[e] / tot;
    } else {
        for (int e = tid; e < E; e += GATE_THREADS) {
            const float s = s_s[e];
            s_s[e] = mode == 1 ? 1.0f / (1.0f + expf(-s)) : sqrtf(s > 20.f ? s : log1pf(expf(s)));
        }
    }
    __syncthreads();
    for (int e = tid; e < E; e += GATE_THREADS) s_b[e] = s_s[e] + (bias ? bias[e] : 0.f);
    __syncthreads();
    for (int k = 0; k < topk; ++k) {
        float bv = -INFINITY;
        int bi = 0x7FFFFFFF;
        for (int e = tid; e < E; e += GATE_THREADS) argmax_pair(bv, bi, s_b[e], e);
        for (int o = 32; o > 0; o >>= 1) {
            const float v2 = __shfl_xor(bv, o);
            const int i2 = __shfl_xor(bi, o);
            argmax_pair(bv, bi, v2, i2);
        }
        if (lane == 0) { s_rv[wave] = bv; s_ri[wave] = bi; }
        __syncthreads();
        if (tid == 0) {
            float v = s_rv[0];
            int i = s_ri[0];
            for (int w = 1; w < GATE_THREADS / WAVE; ++w) argmax_pair(v, i, s_rv[w], s_ri[w]);
            s_i[k] = i;
            s_w[k] = s_s[i];
            s_b[i] = -INFINITY;
        }
        __syncthreads();
    }
    if (tid == 0) {
        float sum = 0.f;
        for (int k = 0; k < topk; ++k) sum += s_w[k];
        for (int k = 0; k < topk; ++k) {
            eid[(long long)row * topk + k] = s_i[k];
            wt[(long long)row * topk + k] = norm ? s_w[k] / (sum + 1e-20f) * route_scale : s_w[k] * route_scale;
        }
    }
}

extern "C" int dsv41_gate_topk(const float* scores, long long lds, const float* bias, int B, int E, float temp, int topk, float route_scale,
                               int score_func, int norm, int* eid, float* wt, void* stream) {
    if (!scores || !eid || !wt || B < 0 || E < 1 || E > GATE_MAX_E || topk < 1 || topk > 32 || topk > E || score_func < 0 || score_func > 2 || lds < E)
        return DSV41_EINVAL;
    if (B == 0) return 0;
    gate_topk_kernel<<<B, GATE_THREADS, 0, (hipStream_t)stream>>>(scores, lds, bias, E, temp, topk, route_scale, score_func, norm, eid, wt);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------------------------------ dispatch
#define DISP_THREADS 1024
#define DISP_WAVES (DISP_THREADS / WAVE)
#define DISP_MAX_E 512

__global__ void __launch_bounds__(DISP_THREADS) moe_dispatch_kernel(const int* __restrict__ eid, const float* __restrict__ wt, int n, int topk,
                                                                    int E, int gmax, int* __restrict__ tok_sorted, float* __restrict__ wt_sorted,
                                                                    int* __restrict__ inv, int* __restrict__ grp_expert, int* __restrict__ grp_start,
                                                                    int* __restrict__ n_groups) {
    __shared__ int s_count[DISP_MAX_E], s_start[DISP_MAX_E], s_cursor[DISP_MAX_E], s_gbase[DISP_MAX_E];
    __shared__ unsigned short s_wcnt[DISP_WAVES][DISP_MAX_E];
    __shared__ int s_scan[DISP_THREADS];
    __shared__ int s_total_groups;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (int e = tid; e < E; e += DISP_THREADS) { s_count[e] = 0; s_cursor[e] = 0; }
    __syncthreads();
    for (int p = tid; p < n; p += DISP_THREADS) {
        const int e = eid[p];
        if (e >= 0 && e < E) atomicAdd(&s_count[e], 1);
    }
    __syncthreads();
    // exclusive scans of counts and group counts over experts: each thread owns a contiguous run of experts
    const int per = (E + DISP_THREADS - 1) / DISP_THREADS;
    const int e0 = tid * per, e1 = min(E, e0 + per);
    int cs = 0, gsum = 0;
    for (int e = e0; e < e1; ++e) { cs += s_count[e]; gsum += (s_count[e] + gmax - 1) / gmax; }
    s_scan[tid] = cs;
    __syncthreads();
    for (int o = 1; o < DISP_THREADS; o <<= 1) {  // Hillis-Steele inclusive scan
        const int v = tid >= o ? s_scan[tid - o] : 0;
        __syncthreads();
        s_scan[tid] += v;
        __syncthreads();
    }
    int run = s_scan[tid] - cs;
    __syncthreads();
    s_scan[tid] = gsum;
    __syncthreads();
    for (int o = 1; o < DISP_THREADS; o <<= 1) {
        const int v = tid >= o ? s_scan[tid - o] : 0;
        __syncthreads();
        s_scan[tid] += v;
        __syncthreads();
    }
    int grun = s_scan[tid] - gsum;
    for (int e = e0; e < e1; ++e) {
        s_start[e] = run;
        s_gbase[e] = grun;
        run += s_count[e];
        grun += (s_count[e] + gmax - 1) / gmax;
    }
    if (tid == DISP_THREADS - 1) s_total_groups = s_scan[tid];
    __syncthreads();
    // stable scatter, one round of DISP_THREADS pairs at a time (E <= 512 for the per-wave count table)
    const unsigned long long below = (lane == 63) ? ~0ull >> 1 : ((1ull << lane) - 1ull);
    for (int base = 0; base < n; base += DISP_THREADS) {
        const int p = base + tid;
        const bool valid = p < n;
        const int e = valid ? eid[p] : -1;
        const bool real = valid && e >= 0 && e < E;
        // rank among this wave's lanes with the same expert, and the wave's count per expert
        int rank = 0, cnt = 0;
        unsigned long long todo = __ballot(real);
        while (todo) {
            const int leader = __ffsll((long long)todo) - 1;
            const int le = __shfl(e, leader);
            const unsigned long long m = __ballot(real && e == le);
            if (real && e == le) { rank = __popcll(m & below); cnt = __popcll(m); }
            todo &= ~m;
        }
        for (int i = tid; i < DISP_WAVES * E; i += DISP_THREADS) s_wcnt[i / E][i % E] = 0;
        __syncthreads();
        if (real && rank == 0) s_wcnt[wave][e] = (unsigned short)cnt;
        __syncthreads();
        if (real) {
            int before = 0;
            for (int w = 0; w < wave; ++w) before += s_wcnt[w][e];
            const int pos = s_start[e] + s_cursor[e] + before + rank;
            tok_sorted[pos] = p / topk;
            wt_sorted[pos] = wt ? wt[p] : 1.f;
            inv[p] = pos;
        }
        __syncthreads();
        for (int ee = tid; ee < E; ee += DISP_THREADS) {
            int add = 0;
            for (int w = 0; w < DISP_WAVES; ++w) add += s_wcnt[w][ee];
            s_cursor[ee] += add;
        }
        __syncthreads();
    }
    // groups of <= gmax pairs per expert, then padding (p2p.cu:124-131)
    for (int e = tid; e < E; e += DISP_THREADS) {
        const int ng = (s_count[e] + gmax - 1) / gmax;
        for (int g = 0; g < ng; ++g) { grp_expert[s_gbase[e] + g] = e; grp_start[s_gbase[e] + g] = s_start[e] + g * gmax; }
    }
    const int G = s_total_groups;
    for (int g = G + tid; g < n; g += DISP_THREADS) { grp_expert[g] = -1; grp_start[g] = n; }
    if (tid == 0) {
        grp_start[G] = n;
        grp_start[n] = n;
        if (n_groups) *n_groups = G;
    }
}

extern "C" int dsv41_moe_dispatch(const int* eid, const float* wt, int n, int topk, int E, int gmax, int* tok_sorted, float* wt_sorted,
                                  int* inv, int* grp_expert, int* grp_start, int* n_groups, void* stream) {
    if (!eid || !tok_sorted || !wt_sorted || !inv || !grp_expert || !grp_start || n < 0 || topk < 1 || E < 1 || E > 512 || gmax < 1)
        return DSV41_EINVAL;
    moe_dispatch_kernel<<<1, DISP_THREADS, 0, (hipStream_t)stream>>>(eid, wt, n, topk, E, gmax, tok_sorted, wt_sorted, inv, grp_expert, grp_start, n_groups);
    return (int)hipGetLastError();
}
