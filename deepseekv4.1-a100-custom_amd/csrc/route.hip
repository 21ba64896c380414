// Routing kernels: the MoE gate (fused2.gate_topk, fused2.py:418-471; model.MoE.gate, model.py:391-404) and the
// expert bucketing of (token, expert) pairs (cukern.moe_dispatch -> p2p.cu:90-132).
//
// gate_topk_kernel: one workgroup per token row. Scores -> softmax / sigmoid / sqrt(softplus), + bias for the
// selection only, TOPK rounds of a block-wide arg-max (lowest index wins ties, fused2.py:441), weights
// renormalised (+1e-20) and scaled.
// moe_dispatch_kernel: one workgroup per 1024 pairs. Histogram (LDS atomics), exclusive scan over experts, then a
// STABLE scatter: pairs keep ascending pair order within an expert (the reference's order is arbitrary,
// p2p.cu:91-93; a stable order makes the tables reproducible); within a wave the rank among same-expert lanes
// comes from ballots, across waves from per-wave counts in LDS.
#include "common.h"
#include "gate.h"

#define GATE_MAX_PER_LANE 32   // E <= 2048 scores per row, held in registers (32 per lane)

template <int PER>
__global__ void __launch_bounds__(64) gate_topk_kernel(const float* __restrict__ scores, long long lds, int nparts, long long pstride,
                                                       const float* __restrict__ bias, int E, float temp, int topk, float route_scale,
                                                       int mode, int norm, int* __restrict__ eid, float* __restrict__ wt) {
    int ki;
    float kw;
    gate_row_wave<PER>(scores + (long long)blockIdx.x * lds, nparts, pstride, bias, E, temp, topk, route_scale, mode, norm, &ki, &kw);
    if (threadIdx.x < topk) {
        eid[(long long)blockIdx.x * topk + threadIdx.x] = ki;
        wt[(long long)blockIdx.x * topk + threadIdx.x] = kw;
    }
}

extern "C" int dsv41_gate_topk(const float* scores, long long lds, const float* bias, int B, int E, float temp, int topk, float route_scale,
                               int score_func, int norm, int* eid, float* wt, int nparts, long long part_stride, void* stream) {
    if (!scores || !eid || !wt || B < 0 || E < 1 || E > 64 * GATE_MAX_PER_LANE || topk < 1 || topk > 64 || topk > E || score_func < 0 ||
        score_func > 2 || lds < E || nparts < 1 || (nparts > 1 && part_stride < (long long)B * lds))
        return DSV41_EINVAL;
    if (B == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
#define GATE_LAUNCH(PER) \
    gate_topk_kernel<PER><<<B, 64, 0, st>>>(scores, lds, nparts, part_stride, bias, E, temp, topk, route_scale, score_func, norm, eid, wt)
    if (E <= 64 * 4) GATE_LAUNCH(4);
    else if (E <= 64 * 6) GATE_LAUNCH(6);
    else if (E <= 64 * 8) GATE_LAUNCH(8);
    else GATE_LAUNCH(GATE_MAX_PER_LANE);
#undef GATE_LAUNCH
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------------------------------ dispatch
#define DISP_THREADS 1024
#define DISP_WAVES (DISP_THREADS / WAVE)
#define DISP_MAX_E 512

// exclusive scan of v over the block's threads (fixed order); the block total lands in *total
__device__ __forceinline__ int block_exclusive_scan(int v, int* s_scan, int* total) {
    const int tid = threadIdx.x;
    s_scan[tid] = v;
    __syncthreads();
    for (int o = 1; o < DISP_THREADS; o <<= 1) {   // Hillis-Steele inclusive scan
        const int t = tid >= o ? s_scan[tid - o] : 0;
        __syncthreads();
        s_scan[tid] += t;
        __syncthreads();
    }
    const int incl = s_scan[tid];
    *total = s_scan[DISP_THREADS - 1];
    __syncthreads();
    return incl - v;
}

// Workgroup b places the pairs of chunk b = [b * 1024, b * 1024 + 1024). It reads every expert id (a few tens of
// KB, L2-resident) to histogram both all pairs and the pairs before its chunk, so each workgroup knows where its
// pairs go without a second launch or scratch memory: pos = start[e] + (pairs of e before the chunk) + (rank of
// the pair among the chunk's pairs of e), ranks from ballots within a wave and per-wave counts across waves.
// Workgroup 0 also writes the group tables.
__global__ void __launch_bounds__(DISP_THREADS) moe_dispatch_kernel(const int* __restrict__ eid, const float* __restrict__ wt, int n, int topk,
                                                                    int E, int gmax, int* __restrict__ tok_sorted, float* __restrict__ wt_sorted,
                                                                    int* __restrict__ inv, int* __restrict__ grp_expert, int* __restrict__ grp_start,
                                                                    int* __restrict__ n_groups) {
    __shared__ int s_count[DISP_MAX_E], s_before[DISP_MAX_E], s_start[DISP_MAX_E], s_gbase[DISP_MAX_E];
    __shared__ unsigned short s_wcnt[DISP_WAVES][DISP_MAX_E];
    __shared__ int s_scan[DISP_THREADS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c0 = blockIdx.x * DISP_THREADS;
    for (int e = tid; e < E; e += DISP_THREADS) { s_count[e] = 0; s_before[e] = 0; }
    for (int i = tid; i < DISP_WAVES * E; i += DISP_THREADS) s_wcnt[i / E][i % E] = 0;
    __syncthreads();
    for (int p = tid; p < n; p += DISP_THREADS) {
        const int e = eid[p];
        if (e >= 0 && e < E) {
            atomicAdd(&s_count[e], 1);
            if (p < c0) atomicAdd(&s_before[e], 1);
        }
    }
    __syncthreads();
    // exclusive scans of the counts and of the group counts over experts: thread t owns a contiguous run
    const int per = (E + DISP_THREADS - 1) / DISP_THREADS;
    const int e0 = tid * per, e1 = min(E, e0 + per);
    int cs = 0, gsum = 0;
    for (int e = e0; e < e1; ++e) { cs += s_count[e]; gsum += (s_count[e] + gmax - 1) / gmax; }
    int total_pairs, total_groups;
    int run = block_exclusive_scan(cs, s_scan, &total_pairs);
    int grun = block_exclusive_scan(gsum, s_scan, &total_groups);
    for (int e = e0; e < e1; ++e) {
        s_start[e] = run;
        s_gbase[e] = grun;
        run += s_count[e];
        grun += (s_count[e] + gmax - 1) / gmax;
    }
    __syncthreads();
    // stable scatter of this chunk
    const unsigned long long below = (lane == 63) ? ~0ull >> 1 : ((1ull << lane) - 1ull);
    const int p = c0 + tid;
    const bool valid = p < n;
    const int e = valid ? eid[p] : -1;
    const bool real = valid && e >= 0 && e < E;
    int rank = 0, cnt = 0;
    unsigned long long todo = __ballot(real);
    while (todo) {
        const int leader = __ffsll((long long)todo) - 1;
        const int le = __shfl(e, leader);
        const unsigned long long m = __ballot(real && e == le);
        if (real && e == le) { rank = __popcll(m & below); cnt = __popcll(m); }
        todo &= ~m;
    }
    if (real && rank == 0) s_wcnt[wave][e] = (unsigned short)cnt;
    __syncthreads();
    if (real) {
        int before = 0;
        for (int w = 0; w < wave; ++w) before += s_wcnt[w][e];
        const int pos = s_start[e] + s_before[e] + before + rank;
        tok_sorted[pos] = p / topk;
        wt_sorted[pos] = wt ? wt[p] : 1.f;
        inv[p] = pos;
    }
    if (valid && !real) inv[p] = -1;   // a dropped pair (id outside [0, E)) has no sorted slot
    if (blockIdx.x != 0) return;
    // groups of <= gmax pairs per expert, then padding (p2p.cu:124-131). The padding starts at the number of
    // placed pairs (n when every id is valid, as in the reference), so the last group ends there; the sorted slots
    // past it (left by dropped pairs) hold token 0 with weight 0.
    for (int ee = tid; ee < E; ee += DISP_THREADS) {
        const int ng = (s_count[ee] + gmax - 1) / gmax;
        for (int g = 0; g < ng; ++g) { grp_expert[s_gbase[ee] + g] = ee; grp_start[s_gbase[ee] + g] = s_start[ee] + g * gmax; }
    }
    const int G = total_groups;
    for (int g = G + tid; g < n; g += DISP_THREADS) { grp_expert[g] = -1; grp_start[g] = total_pairs; }
    for (int q = total_pairs + tid; q < n; q += DISP_THREADS) { tok_sorted[q] = 0; wt_sorted[q] = 0.f; }
    if (tid == 0) {
        grp_start[G] = total_pairs;
        grp_start[n] = total_pairs;
        if (n_groups) *n_groups = G;
    }
}

extern "C" int dsv41_moe_dispatch(const int* eid, const float* wt, int n, int topk, int E, int gmax, int* tok_sorted, float* wt_sorted,
                                  int* inv, int* grp_expert, int* grp_start, int* n_groups, void* stream) {
    if (!eid || !tok_sorted || !wt_sorted || !inv || !grp_expert || !grp_start || n < 0 || topk < 1 || E < 1 || E > 512 || gmax < 1)
        return DSV41_EINVAL;
    const int blocks = n > 0 ? (n + DISP_THREADS - 1) / DISP_THREADS : 1;   // one workgroup writes the (empty) tables when n == 0
    moe_dispatch_kernel<<<blocks, DISP_THREADS, 0, (hipStream_t)stream>>>(eid, wt, n, topk, E, gmax, tok_sorted, wt_sorted, inv, grp_expert, grp_start,
                                                                          n_groups);
    return (int)hipGetLastError();
}
