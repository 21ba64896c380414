// Prefill expert GEMMs on gfx950 block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4), for many tokens per
// expert (model.MoE.__call__ beyond 16 tokens, model.py:539-551, 584-589; moe_kernels.grouped_fp4_gemm,
// moe_kernels.py:127-200).
//
// The (token, expert) pairs arrive bucketed by expert in groups of <= 128 pairs (moe_dispatch tables, gmax 128).
// One workgroup computes a 128-row x 128-pair tile of one group over the full K:
//   MODE 0 (w13): rows = 64 gate rows c0 .. c0 + 63 and the matching 64 up rows I + c0 .., so the epilogue turns
//          the tile into h = fq8(bf16(w * silu(min(g, L)) * clamp(u, +-L))) for 64 columns (two FP8 groups) of
//          every pair (fused.py:284-306) -- gate/up never reach HBM;
//   MODE 1 (w2):  rows = 128 consecutive output rows; the epilogue stores fp32 y2[pair][row].
// 8 waves: wave w owns row blocks (w & 3) and 4 + (w & 3) (a gate block and its up block in MODE 0) and the 64
// pairs of half w >> 2, i.e. 2 x 4 MFMA accumulators. Per 128-k step a wave issues 8 MFMAs; the weight operand
// (raw E2M1 nibbles + E8M0 bytes, as stored) streams from HBM through a PF-deep register ring, the activation
// operand (E4M3 codes of the 128 pairs' tokens, gathered by token id) is staged into a double-buffered LDS tile
// by all 512 threads from the same ring.
// Workgroup order is XCD-aware: the hardware hands workgroup i to XCD i % 8, so the linear id is remapped such
// that each XCD walks its share of (column block, group) items group-fastest. Consecutive groups of one expert
// (a popular expert has many) then run together on one XCD and read each weight tile from that XCD's L2.
#include "common.h"

#define PG_THREADS 512
#define PG_T 128                // pairs per tile
#define PG_LDB (128 + 16)       // LDS row stride of a staged 128-k activation chunk (bytes)
#define PG_PF 2                 // k-steps in flight

struct PrefillArgs {
    const uint8_t* xc; long long ldx;        // E4M3 codes [rows][ldx]: activations (MODE 0) or h (MODE 1)
    const uint8_t* xs; long long ldxs;       // E8M0 [rows][ldxs]
    const uint8_t* W; long long stride_we;   // packed E2M1 [E][N][K/2] (tiled or row-major)
    const uint8_t* S; long long stride_se;
    int N, K, E;                              // N = weight rows (MODE 0: 2 I), K = reduction length
    const int* grp_expert; const int* grp_start; int G;
    const int* row_of_pair;                  // MODE 0: token row of sorted pair p; MODE 1: NULL (row p)
    const float* wt_sorted;                  // MODE 0: routing weight of sorted pair p
    float limit;
    uint8_t* hc; long long ldhc; uint8_t* hs; long long ldhs;   // MODE 0 outputs
    float* y; long long ldy;                                     // MODE 1 output fp32 [pairs][ldy]
    int n_cb;                                 // column blocks (MODE 0: I / 64, MODE 1: N / 128)
    int g_pad;                                // G rounded up to a multiple of 8 (XCD remap)
};

template <int MODE, int TILED>
__global__ void __launch_bounds__(PG_THREADS, 2) prefill_gemm_kernel(const PrefillArgs a) {
    __shared__ __align__(16) uint8_t s_b[2][PG_T][PG_LDB];
    __shared__ uint32_t s_bs[2][PG_T];           // E8M0 bytes of the k-step's four 32-k blocks, per pair
    __shared__ int s_row[PG_T];
    __shared__ float s_amax[8][64];

    // ---- XCD-aware item: each XCD walks a contiguous range of (column block, group) items, group fastest
    const int L = blockIdx.x;
    const int per_xcd = gridDim.x / 8;
    const int item = (L & 7) * per_xcd + (L >> 3);
    const int g = item % a.g_pad, cb = item / a.g_pad;
    if (g >= a.G || cb >= a.n_cb) return;
    const int e = a.grp_expert[g];
    if (e < 0 || e >= a.E) return;
    const int p0 = a.grp_start[g], m = a.grp_start[g + 1] - p0;
    if (m <= 0) return;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rsel = wave & 3, half = wave >> 2;
    const int col = lane & 15, kb = lane >> 4;
    const int K = a.K, nk = K >> 7, Kh = K >> 1, Ks = K >> 5;
    // this wave's two 16-row weight blocks
    int nbA, nbB;
    if (MODE == 0) {
        const int I = a.N >> 1;
        nbA = (cb * 64 + 16 * rsel) >> 4;
        nbB = (I + cb * 64 + 16 * rsel) >> 4;
    } else {
        nbA = (cb * 128 + 16 * rsel) >> 4;
        nbB = nbA + 4;
    }
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.W + (long long)e * a.stride_we, (uint32_t)a.stride_we);
    const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.S + (long long)e * a.stride_se, (uint32_t)a.stride_se);
    const uint32_t wA = (uint32_t)wtile_off<TILED>(nbA, 0, nk, Kh, lane), wB = (uint32_t)wtile_off<TILED>(nbB, 0, nk, Kh, lane);
    const uint32_t sA = (uint32_t)stile_off<TILED>(nbA, 0, nk, Ks, lane), sB = (uint32_t)stile_off<TILED>(nbB, 0, nk, Ks, lane);
    const int ws = TILED ? 1024 : 64, ss = TILED ? 64 : 4;

    // pair rows of the tile (pairs past the group repeat its first row; their results are not stored)
    if (tid < PG_T) {
        const int p = p0 + (tid < m ? tid : 0);
        s_row[tid] = MODE == 0 ? a.row_of_pair[p] : p;
    }
    __syncthreads();
    // staging: thread tid moves 32 bytes (k quarter q) of pair row r; threads with q == 0 also the 4 E8M0 bytes
    const int sr_ = tid >> 2, sq = tid & 3;
    const uint8_t* xsrc = a.xc + (long long)s_row[sr_] * a.ldx + sq * 32;
    const uint8_t* ssrc = a.xs + (long long)s_row[sr_] * a.ldxs;

    v4i RA[PG_PF], RB[PG_PF], X0[PG_PF], X1[PG_PF];
    int SA_[PG_PF], SB_[PG_PF];
    uint32_t XS[PG_PF];
    auto load = [&](int slot, int kc) {
        RA[slot] = buffer_load_tile(wr, wA, (uint32_t)(kc * ws));
        RB[slot] = buffer_load_tile(wr, wB, (uint32_t)(kc * ws));
        SA_[slot] = buffer_load_byte(sr, sA, (uint32_t)(kc * ss));
        SB_[slot] = buffer_load_byte(sr, sB, (uint32_t)(kc * ss));
        X0[slot] = *(const v4i*)(xsrc + kc * 128);
        X1[slot] = *(const v4i*)(xsrc + kc * 128 + 16);
        XS[slot] = sq == 0 ? *(const uint32_t*)(ssrc + kc * 4) : 0u;
    };
    auto stage = [&](int slot, int buf) {
        *(v4i*)&s_b[buf][sr_][sq * 32] = X0[slot];
        *(v4i*)&s_b[buf][sr_][sq * 32 + 16] = X1[slot];
        if (sq == 0) s_bs[buf][sr_] = XS[slot];
    };
    v4f accA[4], accB[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) { accA[t] = v4f{0.f, 0.f, 0.f, 0.f}; accB[t] = accA[t]; }
    int kstep = 0;   // k-step being consumed (slot = kstep % PG_PF)
    auto use = [&](int slot) {
        const int buf = kstep & 1;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int pr = half * 64 + t * 16 + col;
            const v4i b0 = *(const v4i*)&s_b[buf][pr][kb * 16];
            const v4i b1 = *(const v4i*)&s_b[buf][pr][64 + kb * 16];
            const int sb = (int)(s_bs[buf][pr] >> (8 * kb));
            const v8i bv = v8i{b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
            accA[t] = mfma_fp4w_fp8x(v8i{RA[slot].x, RA[slot].y, RA[slot].z, RA[slot].w, 0, 0, 0, 0}, bv, accA[t], SA_[slot], sb);
            accB[t] = mfma_fp4w_fp8x(v8i{RB[slot].x, RB[slot].y, RB[slot].z, RB[slot].w, 0, 0, 0, 0}, bv, accB[t], SB_[slot], sb);
        }
        // the next k-step's activations (loaded PF - 1 steps ago) into the other buffer, which every wave
        // finished reading before the previous barrier
        if (kstep + 1 < nk) stage((slot + 1) % PG_PF, buf ^ 1);
        __syncthreads();
        ++kstep;
    };
    // nk >= PG_PF (checked by the host): the prologue puts steps 0 .. PG_PF - 1 in flight
    pipeline_start<PG_PF>(nk, load);
    stage(0, 0);
    __syncthreads();
    pipeline_finish<PG_PF>(nk, load, use);

    // ---- epilogue
    if (MODE == 0) {
        // lane (col, kb) of wave w holds, for pair half * 64 + 16 t + col, rows 4 kb .. 4 kb + 3 of its gate block
        // (accA) and up block (accB): SwiGLU columns c0 + 16 rsel + 4 kb + i
        const int I = a.N >> 1;
        float h[4][4];
        float am[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int pr = half * 64 + t * 16 + col;
            const float wgt = pr < m ? a.wt_sorted[p0 + pr] : 0.f;
            const float gv[4] = {accA[t].x, accA[t].y, accA[t].z, accA[t].w};
            const float uv[4] = {accB[t].x, accB[t].y, accB[t].z, accB[t].w};
            float mx = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float gg = gv[i], uu = uv[i];
                if (a.limit > 0.f) {
                    uu = fminf(fmaxf(uu, -a.limit), a.limit);
                    gg = fminf(gg, a.limit);
                }
                float hv = gg * (1.0f / (1.0f + expf(-gg))) * uu;
                hv = bf16_round(hv * wgt);
                h[t][i] = hv;
                mx = fmaxf(mx, fabsf(hv));
            }
            // max over the 16 rows of this wave: the 4 lanes holding column col (kb = 0..3)
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            am[t] = mx;
        }
        // one FP8 group = 32 columns = the 16 rows of this wave and of its partner (rsel ^ 1)
        if (kb == 0) {
#pragma unroll
            for (int t = 0; t < 4; ++t) s_amax[wave][t * 16 + col] = am[t];
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int pr = half * 64 + t * 16 + col;
            const float gmax = fmaxf(am[t], s_amax[wave ^ 1][t * 16 + col]);
            const int ex = fq8_exponent(gmax);
            if (pr < m) {
                const long long p = p0 + pr;
                uint32_t codes = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) codes |= fq8_code(h[t][i], ex) << (8 * i);
                const int c = cb * 64 + 16 * rsel + 4 * kb;
                *(uint32_t*)(a.hc + p * a.ldhc + c) = codes;
                if ((rsel & 1) == 0 && kb == 0) a.hs[p * a.ldhs + (c >> 5)] = (uint8_t)(ex + 127);
            }
        }
        (void)I;
    } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int pr = half * 64 + t * 16 + col;
            if (pr < m) {
                float* o = a.y + (long long)(p0 + pr) * a.ldy;
                *(v4f*)(o + nbA * 16 + 4 * kb) = accA[t];
                *(v4f*)(o + nbB * 16 + 4 * kb) = accB[t];
            }
        }
    }
}

// y[t][n] = bf16(sum_j y2[inv[t * topk + j]][n] (+ ys[t][n])), j ascending (model.py:589-591: view(n, k, dim).sum(1)
// then + shared, fp32); optional fp32 y32. One thread per 4 consecutive n.
__global__ void __launch_bounds__(256) combine_pairs_kernel(const float* __restrict__ y2, long long ldy2, const int* __restrict__ inv,
                                                            int topk, int T, int N, const uint16_t* __restrict__ ys, long long ldys,
                                                            uint16_t* __restrict__ out, long long ldo, float* __restrict__ y32, long long ld32) {
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int nq = N >> 2;
    if (idx >= (long long)T * nq) return;
    const int t = (int)(idx / nq), n = (int)(idx - (long long)t * nq) * 4;
    v4f s = v4f{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < topk; ++j) {
        const int r = inv[t * topk + j];
        s += *(const v4f*)(y2 + (long long)r * ldy2 + n);
    }
    if (y32) *(v4f*)(y32 + (long long)t * ld32 + n) = s;
    if (out) {
        const float v[4] = {s.x, s.y, s.z, s.w};
        uint32_t o[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            float a0 = v[2 * i], a1 = v[2 * i + 1];
            if (ys) {
                a0 += bf16_to_f32(ys[(long long)t * ldys + n + 2 * i]);
                a1 += bf16_to_f32(ys[(long long)t * ldys + n + 2 * i + 1]);
            }
            o[i] = f32_to_bf16_bits(a0) | (f32_to_bf16_bits(a1) << 16);
        }
        *(uint2*)(out + (long long)t * ldo + n) = make_uint2(o[0], o[1]);
    }
}

static int launch_prefill(PrefillArgs& a, int mode, int tiled, hipStream_t st) {
    a.g_pad = (a.G + 7) & ~7;
    const long long items = (long long)a.n_cb * a.g_pad;   // a multiple of 8
    if (items > 0x7FFFFFFFll) return DSV41_EINVAL;
    const dim3 grid((unsigned)items), block(PG_THREADS);
    if (mode == 0) { if (tiled) prefill_gemm_kernel<0, 1><<<grid, block, 0, st>>>(a); else prefill_gemm_kernel<0, 0><<<grid, block, 0, st>>>(a); }
    else { if (tiled) prefill_gemm_kernel<1, 1><<<grid, block, 0, st>>>(a); else prefill_gemm_kernel<1, 0><<<grid, block, 0, st>>>(a); }
    return (int)hipGetLastError();
}

extern "C" int dsv41_prefill_up(const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, const uint8_t* W13, long long stride_we,
                                const uint8_t* S13, long long stride_se, int tiled, int E, int H, int I, const int* grp_expert,
                                const int* grp_start, int G, const int* tok_sorted, const float* wt_sorted, float limit, uint8_t* hc,
                                long long ldhc, uint8_t* hs, long long ldhs, void* stream) {
    if (!xc || !xs || !W13 || !S13 || !grp_expert || !grp_start || !tok_sorted || !wt_sorted || !hc || !hs) return DSV41_EINVAL;
    if (E < 1 || H < 128 * PG_PF || (H & 127) || I <= 0 || (I & 63) || G < 0 || ldx < H || (ldx & 15) || (((uintptr_t)xc) & 15) || ldxs < H / 32 ||
        (ldxs & 3) || (((uintptr_t)xs) & 3) || ldhc < I || (ldhc & 3) || (((uintptr_t)hc) & 3) || ldhs < I / 32)
        return DSV41_EINVAL;
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll || stride_we < (long long)2 * I * (H / 2) ||
        stride_se < (long long)2 * I * (H / 32))
        return DSV41_EINVAL;
    if (G == 0) return 0;
    PrefillArgs a{xc, ldx, xs, ldxs, W13, stride_we, S13, stride_se, 2 * I, H, E, grp_expert, grp_start, G, tok_sorted, wt_sorted, limit,
                  hc, ldhc, hs, ldhs, nullptr, 0, I / 64, 0};
    return launch_prefill(a, 0, tiled, (hipStream_t)stream);
}

extern "C" int dsv41_prefill_down(const uint8_t* hc, long long ldhc, const uint8_t* hs, long long ldhs, const uint8_t* W2, long long stride_we,
                                  const uint8_t* S2, long long stride_se, int tiled, int E, int H, int I, const int* grp_expert,
                                  const int* grp_start, int G, float* y2, long long ldy, void* stream) {
    if (!hc || !hs || !W2 || !S2 || !grp_expert || !grp_start || !y2) return DSV41_EINVAL;
    if (E < 1 || H <= 0 || (H & 127) || I < 128 * PG_PF || (I & 127) || G < 0 || ldhc < I || (ldhc & 15) || (((uintptr_t)hc) & 15) || ldhs < I / 32 ||
        (ldhs & 3) || (((uintptr_t)hs) & 3) || ldy < H || (ldy & 3) || (((uintptr_t)y2) & 15))
        return DSV41_EINVAL;
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll || stride_we < (long long)H * (I / 2) ||
        stride_se < (long long)H * (I / 32))
        return DSV41_EINVAL;
    if (G == 0) return 0;
    PrefillArgs a{hc, ldhc, hs, ldhs, W2, stride_we, S2, stride_se, H, I, E, grp_expert, grp_start, G, nullptr, nullptr, 0.f,
                  nullptr, 0, nullptr, 0, y2, ldy, H / 128, 0};
    return launch_prefill(a, 1, tiled, (hipStream_t)stream);
}

extern "C" int dsv41_combine_pairs(const float* y2, long long ldy2, const int* inv, int topk, int T, int N, const uint16_t* ys, long long ldys,
                                   uint16_t* out, long long ldo, float* y32, long long ld32, void* stream) {
    if (!y2 || !inv || topk < 1 || T < 0 || N <= 0 || (N & 3) || ldy2 < N || (ldy2 & 3) || (((uintptr_t)y2) & 15) || (!out && !y32) ||
        (out && (ldo < N || (ldo & 3) || (((uintptr_t)out) & 7))) || (y32 && (ld32 < N || (ld32 & 3) || (((uintptr_t)y32) & 15))) ||
        (ys && ldys < N))
        return DSV41_EINVAL;
    if (T == 0) return 0;
    const long long n = (long long)T * (N / 4);
    combine_pairs_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(y2, ldy2, inv, topk, T, N, ys, ldys, out, ldo, y32, ld32);
    return (int)hipGetLastError();
}
