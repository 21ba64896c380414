// Grouped FP4 expert GEMV/GEMM on gfx950 block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// The weights are consumed as stored: E2M1 nibbles and their E8M0 bytes go straight into the MFMA A operand
// and its scale operand, so no instruction decodes a weight. The activations are FP8 E4M3 codes with E8M0
// bytes per 32 (what fake_quant_fp8 / swiglu_quant produce, exactly), fed as the B operand. One MFMA consumes
// a 16-row x 128-k weight tile = 1 KiB; both supported layouts make that tile one contiguous 1 KiB block
// (tile_fp4) or 16 contiguous 64 B row pieces (row-major), so every wave-wide weight load is fully used.
//
// Kernels:
//  fp4_grouped_kernel  out[p, n] = wt[p] * sum_k x[pair_tok[p], k] * deq(W[e_g])[n, k]  for pairs p of group g
//                      (cukern.fp4_gemm_tc / fp4_gemv_pairs / moe_kernels.grouped_fp4_gemm semantics,
//                      cukern.py:60-77, 238-276; moe_kernels.py:127-151). One wave = one (group, 16-row block);
//                      up to 16*NCH pairs share each weight tile (one MFMA per 16 pairs).
//  moe_down_sum_kernel y[t, n] = sum over groups g, pairs p of g with token t: h_p . deq(W2[e_g])[n, :]
//                      (decode w2 + the fixed per-token sum of decode.py:316-335 / fused2.py:490-495): the
//                      B column is the token, so all experts of a token accumulate in one MFMA accumulator and
//                      every selected expert's w2 is read once. Optional epilogue: bf16(y + shared-expert ys).
#include "common.h"

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

__device__ __forceinline__ v8i widen(v4i a) { return v8i{a.x, a.y, a.z, a.w, 0, 0, 0, 0}; }
__device__ __forceinline__ v8i join(v4i a, v4i b) { return v8i{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}; }

struct GroupedArgs {
    const uint8_t* W; long long stride_we;   // [E][N][K/2] packed E2M1 (expert stride in bytes)
    const uint8_t* S; long long stride_se;   // [E][N][K/32] E8M0
    int N, K;
    const uint8_t* xc; long long ldx;        // FP8 codes [rows][K], row stride in bytes
    const uint8_t* xs; long long ldxs;       // E8M0 [rows][K/32], row stride in bytes
    const int* grp_expert; const int* grp_start; const int* pair_tok;
    float* out; long long ldo;               // fp32 [rows][ldo]
    const int* out_row;                      // optional: output row of pair p (default p)
    const float* pair_wt;                    // optional per-pair factor
    int shard_start, shard_n, zero_out, min_tok, max_tok, vec_store;
    int accum;                               // 0 store, 1 add (distinct rows), 2 atomic add (rows may repeat)
};

template <int NCH, int TILED, int PF>
__global__ void __launch_bounds__(256) fp4_grouped_kernel(const GroupedArgs a) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = blockIdx.x * 4 + wave;
    const int g = blockIdx.y;
    if (nb * 16 >= a.N) return;
    const int p0 = a.grp_start[g], p1 = a.grp_start[g + 1];
    const int m = p1 - p0;
    if (m <= 0 || m < a.min_tok || m > a.max_tok) return;
    const int col = lane & 15, kb = lane >> 4;
    const int row0 = nb * 16 + 4 * kb;   // this lane's 4 output rows
    const int e = a.grp_expert[g] - a.shard_start;
    if (e < 0 || e >= a.shard_n) {       // another GPU's expert (cukern.py:244-246): skip, optionally zero
        if (a.zero_out && a.accum == 0)
            for (int q = p0 + col; q < p1; q += 16) {
                const long long orow = a.out_row ? a.out_row[q] : q;
#pragma unroll
                for (int i = 0; i < 4; ++i) a.out[orow * a.ldo + row0 + i] = 0.f;
            }
        return;
    }
    const int nk = a.K >> 7, Kh = a.K >> 1, Ks = a.K >> 5;
    const uint8_t* wbase = a.W + (long long)e * a.stride_we;
    const uint8_t* sbase = a.S + (long long)e * a.stride_se;
    const long long w0 = wtile_off<TILED>(nb, 0, nk, Kh, lane), ws = TILED ? 1024 : 64;
    const long long s0 = stile_off<TILED>(nb, 0, nk, Ks, lane), ss = TILED ? 64 : 4;

    for (int base = p0; base < p1; base += 16 * NCH) {
        const uint8_t* xp[NCH];
        const uint8_t* xsp[NCH];
        bool ok[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int q = base + c * 16 + col;
            ok[c] = q < p1;
            const long long r = ok[c] ? a.pair_tok[q] : 0;
            xp[c] = a.xc + r * a.ldx + kb * 16;
            xsp[c] = a.xs + r * a.ldxs + kb;
        }
        v4f acc[NCH];
#pragma unroll
        for (int c = 0; c < NCH; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};

        v4i A[PF];
        int SA[PF];
        v4i B0[NCH][PF], B1[NCH][PF];
        int SB[NCH][PF];
        auto load = [&](int slot, int kc) {
            A[slot] = __builtin_nontemporal_load((const v4i*)(wbase + w0 + kc * ws));
            SA[slot] = sbase[s0 + kc * ss];
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                if (ok[c]) {
                    const uint8_t* p = xp[c] + kc * 128;
                    B0[c][slot] = *(const v4i*)p;
                    B1[c][slot] = *(const v4i*)(p + 64);
                    SB[c][slot] = xsp[c][kc * 4];
                } else {
                    B0[c][slot] = v4i{0, 0, 0, 0};
                    B1[c][slot] = v4i{0, 0, 0, 0};
                    SB[c][slot] = 127;
                }
            }
        };
#pragma unroll
        for (int i = 0; i < PF; ++i)
            if (i < nk) load(i, i);
        for (int k0 = 0; k0 < nk; k0 += PF) {
#pragma unroll
            for (int i = 0; i < PF; ++i) {
                const int kc = k0 + i;
                if (kc < nk) {
                    const v8i av = widen(A[i]);
#pragma unroll
                    for (int c = 0; c < NCH; ++c) acc[c] = mfma_fp4w_fp8x(av, join(B0[c][i], B1[c][i]), acc[c], SA[i], SB[c][i]);
                    if (kc + PF < nk) load(i, kc + PF);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if (!ok[c]) continue;
            const int q = base + c * 16 + col;
            const float f = a.pair_wt ? a.pair_wt[q] : 1.f;
            float* o = a.out + (a.out_row ? (long long)a.out_row[q] : (long long)q) * a.ldo + row0;
            const v4f v = acc[c] * f;
            if (a.accum == 2) {
                atomicAdd(o + 0, v.x); atomicAdd(o + 1, v.y); atomicAdd(o + 2, v.z); atomicAdd(o + 3, v.w);
            } else if (a.accum == 1) {
                o[0] += v.x; o[1] += v.y; o[2] += v.z; o[3] += v.w;
            } else if (a.vec_store) {
                *(v4f*)o = v;
            } else {
                o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------ decode w2 + sum
struct DownSumArgs {
    const uint8_t* W; long long stride_we;
    const uint8_t* S; long long stride_se;
    int N, K;                                 // N = hidden (output rows), K = intermediate
    const uint8_t* hc; long long ldh;         // FP8 codes of h, pairs in expert-sorted order
    const uint8_t* hs; long long ldhs;
    const int* grp_expert; const int* grp_start; const int* tok_sorted;
    int n_slots;                              // group slots to scan (= pairs); unused slots have expert -1
    int M;                                    // tokens (<= 16)
    float* y; long long ldy;                  // optional fp32 [M][N] routed sum
    const uint16_t* ys; long long ldys;       // optional bf16 shared-expert output
    uint16_t* yb; long long ldyb;             // optional bf16 [M][N] = bf16(y + ys)
    int shard_start, shard_n;
};

#define DS_MAX_SLOTS 256

template <int TILED, int PF>
__global__ void __launch_bounds__(256) moe_down_sum_kernel(const DownSumArgs a) {
    __shared__ int s_exp[DS_MAX_SLOTS];
    __shared__ short s_pair[DS_MAX_SLOTS][16];
    __shared__ int s_ngroups;
    __shared__ v4f s_red[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = blockIdx.x;
    // per-group table: expert (shard-local, -1 = skip) and, per token column, the group's pair (-1 = none)
    if (threadIdx.x == 0) s_ngroups = 0;
    __syncthreads();
    for (int g = threadIdx.x; g < a.n_slots; g += blockDim.x) {
        const int ge = a.grp_expert[g];
        int e = ge < 0 ? -1 : ge - a.shard_start;
        if (e >= a.shard_n) e = -1;
        s_exp[g] = e;
#pragma unroll
        for (int t = 0; t < 16; ++t) s_pair[g][t] = -1;
        if (ge >= 0) {
            atomicMax(&s_ngroups, g + 1);
            for (int q = a.grp_start[g]; q < a.grp_start[g + 1]; ++q) s_pair[g][a.tok_sorted[q] & 15] = (short)q;
        }
    }
    __syncthreads();
    const int G = s_ngroups;
    const int col = lane & 15, kb = lane >> 4;
    const int nk = a.K >> 7, Kh = a.K >> 1, Ks = a.K >> 5;
    const long long w0 = wtile_off<TILED>(nb, 0, nk, Kh, lane), ws = TILED ? 1024 : 64;
    const long long s0 = stile_off<TILED>(nb, 0, nk, Ks, lane), ss = TILED ? 64 : 4;

    // this wave's iteration space: groups g = wave, wave + 4, ... (valid ones) x k-chunks, flattened so the
    // load pipeline runs across group boundaries
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    v4i A[PF], B0[PF], B1[PF];
    int SA[PF], SB[PF];
    int lg = wave, lkc = 0;                   // load cursor: group slot, k-chunk
    while (lg < G && s_exp[lg] < 0) lg += 4;
    auto load = [&](int slot) {
        const int e = s_exp[lg];
        const int q = s_pair[lg][col];
        A[slot] = __builtin_nontemporal_load((const v4i*)(a.W + (long long)e * a.stride_we + w0 + lkc * ws));
        SA[slot] = a.S[(long long)e * a.stride_se + s0 + lkc * ss];
        if (q >= 0) {
            const uint8_t* p = a.hc + (long long)q * a.ldh + lkc * 128 + kb * 16;
            B0[slot] = *(const v4i*)p;
            B1[slot] = *(const v4i*)(p + 64);
            SB[slot] = a.hs[(long long)q * a.ldhs + lkc * 4 + kb];
        } else {
            B0[slot] = v4i{0, 0, 0, 0};
            B1[slot] = v4i{0, 0, 0, 0};
            SB[slot] = 127;
        }
        if (++lkc == nk) {
            lkc = 0;
            lg += 4;
            while (lg < G && s_exp[lg] < 0) lg += 4;
        }
    };
    int total = 0;
    for (int g = wave; g < G; g += 4) total += s_exp[g] >= 0 ? nk : 0;
#pragma unroll
    for (int i = 0; i < PF; ++i)
        if (i < total) load(i);
    for (int k0 = 0; k0 < total; k0 += PF) {
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            const int it = k0 + i;
            if (it < total) {
                acc = mfma_fp4w_fp8x(widen(A[i]), join(B0[i], B1[i]), acc, SA[i], SB[i]);
                if (it + PF < total) load(i);
            }
        }
    }
    s_red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    const v4f sum = ((s_red[0][lane] + s_red[1][lane]) + s_red[2][lane]) + s_red[3][lane];
    if (col >= a.M) return;
    const int row0 = nb * 16 + 4 * kb;
    if (a.y) {
        float* o = a.y + (long long)col * a.ldy + row0;
        o[0] = sum.x; o[1] = sum.y; o[2] = sum.z; o[3] = sum.w;
    }
    if (a.yb) {
        float v[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float t = v[i];
            if (a.ys) t += bf16_to_f32(a.ys[(long long)col * a.ldys + row0 + i]);
            a.yb[(long long)col * a.ldyb + row0 + i] = (uint16_t)f32_to_bf16_bits(t);
        }
    }
}

// ------------------------------------------------------------------------------------------ C ABI
template <int NCH, int TILED>
static void launch_grouped(const GroupedArgs& a, int G, hipStream_t st) {
    dim3 grid((unsigned)((a.N / 16 + 3) / 4), (unsigned)G);
    constexpr int PF = NCH == 1 ? 8 : (NCH == 2 ? 4 : 2);
    fp4_grouped_kernel<NCH, TILED, PF><<<grid, 256, 0, st>>>(a);
}

extern "C" int dsv41_fp4_grouped_gemm(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                                      int N, int K, const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs,
                                      const int* grp_expert, const int* grp_start, int G, const int* pair_tok,
                                      float* out, long long ldo, const int* out_row, const float* pair_wt, int accum, int max_tokens,
                                      int shard_start, int shard_n, int zero_out, int min_tok, int max_tok, void* stream) {
    if (!W || !S || !xc || !xs || !grp_expert || !grp_start || !pair_tok || !out) return DSV41_EINVAL;
    if (N <= 0 || (N & 15) || K <= 0 || (K & 127) || G < 0 || ldo < N || ldx < K || ldxs < K / 32 || max_tokens < 1) return DSV41_EINVAL;
    if (accum < 0 || accum > 2) return DSV41_EINVAL;
    if (G == 0) return 0;
    GroupedArgs a{W, stride_we, S, stride_se, N, K, xc, ldx, xs, ldxs, grp_expert, grp_start, pair_tok, out, ldo, out_row, pair_wt,
                  shard_start, shard_n, zero_out, min_tok, max_tok, 0, accum};
    a.vec_store = ((ldo & 3) == 0 && (((uintptr_t)out) & 15) == 0) ? 1 : 0;
    hipStream_t st = (hipStream_t)stream;
    const int nch = max_tokens <= 16 ? 1 : (max_tokens <= 32 ? 2 : 4);
    if (tiled) {
        if (nch == 1) launch_grouped<1, 1>(a, G, st); else if (nch == 2) launch_grouped<2, 1>(a, G, st); else launch_grouped<4, 1>(a, G, st);
    } else {
        if (nch == 1) launch_grouped<1, 0>(a, G, st); else if (nch == 2) launch_grouped<2, 0>(a, G, st); else launch_grouped<4, 0>(a, G, st);
    }
    return (int)hipGetLastError();
}

extern "C" int dsv41_moe_down_sum(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                                  int N, int K, const uint8_t* hc, long long ldh, const uint8_t* hs, long long ldhs,
                                  const int* grp_expert, const int* grp_start, const int* tok_sorted, int n_slots, int M,
                                  float* y, long long ldy, const uint16_t* ys, long long ldys, uint16_t* yb, long long ldyb,
                                  int shard_start, int shard_n, void* stream) {
    if (!W || !S || !hc || !hs || !grp_expert || !grp_start || !tok_sorted || (!y && !yb)) return DSV41_EINVAL;
    if (N <= 0 || (N & 15) || K <= 0 || (K & 127) || n_slots < 0 || n_slots > DS_MAX_SLOTS || M < 1 || M > 16) return DSV41_EINVAL;
    DownSumArgs a{W, stride_we, S, stride_se, N, K, hc, ldh, hs, ldhs, grp_expert, grp_start, tok_sorted, n_slots, M,
                  y, ldy, ys, ldys, yb, ldyb, shard_start, shard_n};
    hipStream_t st = (hipStream_t)stream;
    if (tiled) moe_down_sum_kernel<1, 8><<<N / 16, 256, 0, st>>>(a);
    else moe_down_sum_kernel<0, 8><<<N / 16, 256, 0, st>>>(a);
    return (int)hipGetLastError();
}
