// Dense FP8 weights times bf16 activations for up to 64 rows: the reference's W8 / linear_w / oproj_a family
// (w8.py:57-124) behind cukern.fp8_gemm_tc and cukern.fp8_gemv (cukern.py:78-218).
//   out[t, n] = sum_k x[t, k] * w[n, k] * 2^(s[n / 32][k / 32] - 127)          fp32 accumulation
// w: float8_e4m3fn bytes [N][K]; s: E8M0 bytes [ceil(N/32)][K/32]. A bf16 activation times an E4M3 weight with a
// power-of-two scale is exact in fp32, as in the reference (exact decode to bf16, fp32 accumulation), so results
// differ from it only in the order of the fp32 additions.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16): the weights are the A operand (16 rows n), the activations the B
// operand (16 tokens). Lane l = 16 j + r holds 16 consecutive weight bytes of row r, k = 16 j .. 16 j + 15 of a
// 64-k chunk, decodes them with their block scale in the converter (v_cvt_scalef32_pk_bf16_fp8; e4m3 x 2^e is
// exact in bf16 over the normal range) and issues two MFMAs, one over the lower 8 k of every lane and one over
// the upper 8. Any fixed assignment of k to MFMA positions is valid while the activation lane holds the same k,
// so the weights need no k permutation (the reference stores a k-permuted order for its mma fragments,
// w8.py:21-37).
// Tiled layout [N/16][K/64][4][16][16 B]: the 16 bytes of lane l sit at byte 16 l of a 1 KiB tile, so a
// wave-load is one contiguous 1 KiB block. Natural layout: row-major with row stride ldw.
// One workgroup per 16-row block; its waves split K and add their partial tiles through LDS in wave order, so the
// result is deterministic and no workgroup waits for another. Every workgroup of a launch is meant to be resident at
// once (<= 128 VGPRs: two 512-thread workgroups per CU), which balances a grid of more row blocks than CUs. A K split
// across workgroups was measured and dropped: publishing partials needs a device-scope release, and its L2 write-back
// made each such workgroup cost microseconds.
#include "common.h"

struct Fp8Args {
    const uint8_t* W; long long ldw;     // bytes per row (natural layout); tiled: ldw == K
    const uint8_t* S; long long lds;     // E8M0 row stride in bytes (one row per 32 weight rows)
    int N, K, nk;                        // nk = K / 64 chunks
    const uint16_t* x; long long ldx;    // bf16 activations
    long long ldt;                       // element stride between the tokens of one output row set
    int M, gc;                           // output rows; gc > 0: row block nb reads x rows offset by (16 nb / gc)
    float* out; long long ldo;           // optional fp32 [M][ldo]
    uint16_t* outb; long long ldob;      // optional bf16 [M][ldob]
};

template <int MT>
__device__ __forceinline__ void fp8_store(const Fp8Args& a, const v4f (&sum)[MT], int n0, int r) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int t = mt * 16 + r;
        if (t >= a.M) continue;
        const float v[4] = {sum[mt].x, sum[mt].y, sum[mt].z, sum[mt].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int n = n0 + i;
            if (n >= a.N) continue;
            if (a.out) a.out[(long long)t * a.ldo + n] = v[i];
            if (a.outb) a.outb[(long long)t * a.ldob + n] = (uint16_t)f32_to_bf16_bits(v[i]);
        }
    }
}

// WPG waves split the workgroup's chunk range; MT 16-token tiles share every weight tile (M <= 16 MT). RB row blocks
// per workgroup (16 RB rows): every activation load a wave makes then feeds RB weight tiles instead of one, so the
// vector memory pipe carries 2 / RB KiB of activations per KiB of weights instead of 2 KiB. Row blocks 2q and 2q + 1
// of a workgroup share their 32-row scale row (the first is even), and a row block past the last one reads the last
// one again and stores nothing. RB > 1 needs gc == 0 or gc % (16 RB) == 0 (one x offset for all the blocks).
template <int WPG, int PF, int MT, int TILED, int RB>
__global__ void __launch_bounds__(WPG * 64) fp8_gemm_kernel(const Fp8Args a) {
    __shared__ v4f s_red[WPG][RB * MT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, j = lane >> 4;
    const int nbt = (a.N + 15) / 16;
    const int nb = blockIdx.x * RB;
    const int c0 = a.nk * wave / WPG, c1 = a.nk * (wave + 1) / WPG;
    const uint8_t* wp[RB];
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        const int nbr = min(nb + b, nbt - 1);
        const int row = min(nbr * 16 + r, a.N - 1);   // rows past N (natural layout) read row N-1, never stored
        wp[b] = TILED ? a.W + ((long long)nbr * a.nk + c0) * 1024 + lane * 16 : a.W + (long long)row * a.ldw + (long long)c0 * 64 + j * 16;
    }
    constexpr long long wstep = TILED ? 1024 : 64;
    constexpr int NS = (RB + 1) / 2;   // 32-row scale rows: row blocks 2q and 2q + 1 of the workgroup share one
    const uint8_t* sp8[NS];
#pragma unroll
    for (int q = 0; q < NS; ++q) sp8[q] = a.S + (long long)(min(nb + 2 * q, nbt - 1) >> 1) * a.lds + 2 * c0 + (j >> 1);
    const long long goff = a.gc ? (long long)((nb * 16) / a.gc) * a.ldx : 0;
    const uint16_t* xp[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int t = min(mt * 16 + r, a.M - 1);   // token columns past M read row M-1, never stored
        xp[mt] = a.x + goff + (long long)t * a.ldt + (long long)c0 * 64 + j * 16;
    }
    v4f acc[RB][MT];
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[b][mt] = v4f{0.f, 0.f, 0.f, 0.f};
    v4i A[PF][RB], X[PF][MT][2];
    int SB[PF][NS];
    pipelined<PF>(c1 - c0,
        [&](int s, int c) {
#pragma unroll
            for (int b = 0; b < RB; ++b) A[s][b] = __builtin_nontemporal_load((const v4i*)(wp[b] + (long long)c * wstep));
#pragma unroll
            for (int q = 0; q < NS; ++q) SB[s][q] = sp8[q][2 * c];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                X[s][mt][0] = *(const v4i*)(xp[mt] + (long long)c * 64);
                X[s][mt][1] = *(const v4i*)(xp[mt] + (long long)c * 64 + 8);
            }
        },
        [&](int s) {
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                v8bf16_t lo, hi;
                decode16(A[s][b], e8m0_to_f32((uint32_t)SB[s][b >> 1]), lo, hi);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    acc[b][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, __builtin_bit_cast(v8bf16_t, X[s][mt][0]), acc[b][mt], 0, 0, 0);
                    acc[b][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, __builtin_bit_cast(v8bf16_t, X[s][mt][1]), acc[b][mt], 0, 0, 0);
                }
            }
        });
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) s_red[wave][b * MT + mt][lane] = acc[b][mt];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int b = 0; b < RB; ++b) {
        if (nb + b >= nbt) break;
        v4f sum[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            sum[mt] = s_red[0][b * MT + mt][lane];
#pragma unroll
            for (int w = 1; w < WPG; ++w) sum[mt] += s_red[w][b * MT + mt][lane];
        }
        const int n0 = (nb + b) * 16 + 4 * j;   // the accumulator of lane l holds rows 4 (l / 16) .. +3, token l % 16
        fp8_store<MT>(a, sum, n0, r);
    }
}

// M <= 4 tokens (every wave owning at least one chunk): each wave first copies its own k range of the activations and of its row block's scale bytes into a
// private LDS region (no barrier: only the wave itself reads it), so the memory pipe carries nothing but the weight
// tiles while it streams them, and the prefetch slots hold weights only (deeper prefetch in fewer registers).
// LDS per wave: M x cpw x 128 B of activations + 2 cpw scale bytes + a 16-byte sink (cpw = chunks per wave, rounded up).
constexpr int FP8_XL_PIECES = 8;   // 16-byte activation pieces per lane: M x chunks per wave <= 64
__host__ __device__ constexpr int fp8_lds_region(int M, int cpw) { return M * cpw * 128 + ((2 * cpw + 15) & ~15) + 16; }

// One wave's part of the LDS-staged GEMV, with exactly P weight tiles in flight: the caller guarantees n >= P, so the
// prologue below is straight-line code and the wait counters track the activation loads exactly (a prologue behind
// a branch makes them wait for every load issued before the merge, draining the weight prefetch).
template <int P, int TILED>
__device__ __forceinline__ v4f fp8_lds_wave(const Fp8Args& a, int cpw, uint8_t* s_dyn, int wave, int lane, int c0, int n) {
    const int r = lane & 15, j = lane >> 4;
    const int nb = blockIdx.x;
    const int xrow = cpw * 64;                                          // bf16 elements per token row in LDS
    const int region = fp8_lds_region(a.M, cpw);
    uint16_t* xl = (uint16_t*)(s_dyn + (size_t)wave * region);
    uint8_t* sl = s_dyn + (size_t)wave * region + a.M * cpw * 128;
    uint8_t* sink = s_dyn + (size_t)wave * region + region - 16;       // target of the writes that carry nothing
    const long long goff = a.gc ? (long long)((nb * 16) / a.gc) * a.ldx : 0;
    // activations -> LDS: piece p of token t covers k = c0 * 64 + 8 q .. + 7 (q = p % (8 n)); every lane loads its
    // pieces first (clamped to a valid address), then stores them; pieces past the end go to the sink (a conditional
    // store would put a branch between the loads and their waits)
    const int per_tok = 8 * n, total = a.M * per_tok;
    v4i xr[FP8_XL_PIECES];
#pragma unroll
    for (int i = 0; i < FP8_XL_PIECES; ++i) {
        const int p = min(lane + 64 * i, total - 1);
        const int t = p / per_tok, q = p - t * per_tok;
        xr[i] = *(const v4i*)(a.x + goff + (long long)t * a.ldt + (long long)c0 * 64 + 8 * q);
    }
    const uint8_t* srow = a.S + (long long)(nb >> 1) * a.lds + 2 * c0;
    const int sb0 = srow[min(lane, 2 * n - 1)], sb1 = srow[min(lane + 64, 2 * n - 1)];
    const uint8_t* wp = TILED ? a.W + ((long long)nb * a.nk + c0) * 1024 + lane * 16
                              : a.W + (long long)min(nb * 16 + r, a.N - 1) * a.ldw + (long long)c0 * 64 + j * 16;
    constexpr long long wstep = TILED ? 1024 : 64;
    v4i A[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        A[i] = __builtin_nontemporal_load((const v4i*)(wp + (long long)i * wstep));
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < FP8_XL_PIECES; ++i) {
        const int p = lane + 64 * i;
        const int t = p / per_tok, q = p - t * per_tok;
        *(v4i*)(p < total ? (uint8_t*)(xl + t * xrow + 8 * q) : sink) = xr[i];
    }
    *(lane < 2 * n ? sl + lane : sink) = (uint8_t)sb0;
    *(lane + 64 < 2 * n ? sl + lane + 64 : sink + 1) = (uint8_t)sb1;
    // other lanes of this wave read what these lanes wrote: keep the LDS reads after the writes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const uint16_t* xt = xl + min(r, a.M - 1) * xrow + j * 16;         // token columns past M repeat row M-1
    const uint8_t* st = sl + (j >> 1);
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    int ci = 0;
    pipeline_finish<P>(n,
        [&](int s, int c) { A[s] = __builtin_nontemporal_load((const v4i*)(wp + (long long)c * wstep)); },
        [&](int s) {
            v8bf16_t lo, hi;
            decode16(A[s], e8m0_to_f32((uint32_t)st[2 * ci]), lo, hi);
            const v4i X0 = *(const v4i*)(xt + ci * 64), X1 = *(const v4i*)(xt + ci * 64 + 8);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, __builtin_bit_cast(v8bf16_t, X0), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, __builtin_bit_cast(v8bf16_t, X1), acc, 0, 0, 0);
            ++ci;
        });
    return acc;
}

template <int WPG, int PF, int TILED>
__global__ void __launch_bounds__(WPG * 64) fp8_gemv_lds_kernel(const Fp8Args a, int cpw) {
    extern __shared__ __align__(16) uint8_t s_dyn[];
    __shared__ v4f s_red[WPG][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c0 = a.nk * wave / WPG, c1 = a.nk * (wave + 1) / WPG, n = c1 - c0;
    const v4f acc = n >= PF ? fp8_lds_wave<PF, TILED>(a, cpw, s_dyn, wave, lane, c0, n)
                  : n >= 4 ? fp8_lds_wave<4, TILED>(a, cpw, s_dyn, wave, lane, c0, n)
                           : fp8_lds_wave<1, TILED>(a, cpw, s_dyn, wave, lane, c0, n);
    s_red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    v4f sum[1] = {s_red[0][lane]};
#pragma unroll
    for (int w = 1; w < WPG; ++w) sum[0] += s_red[w][lane];
    fp8_store<1>(a, sum, blockIdx.x * 16 + 4 * (lane >> 4), lane & 15);
}

// ------------------------------------------------------------------------------------------ dequantisation
// Exact fp32 bit pattern of E4M3 code c times 2^(b-127), as quant.dequant_fp8_block computes it in fp32
// (quant.py:90-95): w.float() * 2^(b-127) with IEEE rounding where the product is subnormal. Byte 255 is +inf.
__device__ __forceinline__ uint32_t e4m3_e8m0_f32_bits(uint32_t c, uint32_t b) {
    const uint32_t sign = (c & 0x80u) << 24;
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    if (e == 15u && m == 7u) return sign | 0x7FC00000u;            // NaN code
    const uint32_t M = e ? (8u | m) : m;                            // value = M * 2^(E + b - 127)
    const int E = (int)(e ? e : 1u) - 10;
    if (b == 255u) return M ? (sign | 0x7F800000u) : 0xFFC00000u;   // x inf (0 x inf = NaN)
    if (M == 0u) return sign;
    const int h = 31 - __builtin_clz(M);                            // 0..3
    const int biased = h + E + (int)b;                              // biased fp32 exponent of the product
    if (biased >= 255) return sign | 0x7F800000u;
    if (biased >= 1) return sign | ((uint32_t)biased << 23) | ((M << (23 - h)) & 0x7FFFFFu);
    const int sh = E + (int)b + 22;                                 // subnormal: M * 2^sh units of 2^-149
    if (sh >= 0) return sign | (M << sh);
    if (sh < -5) return sign;                                       // below half the smallest subnormal
    const uint32_t q = M >> (-sh), rem = M & ((1u << (-sh)) - 1u), half = 1u << (-sh - 1);
    return sign | (q + ((rem > half || (rem == half && (q & 1u))) ? 1u : 0u));
}

// one thread per 16 weights of a row: 16 B in, 32 B out (natural row-major bf16)
__global__ void dequant_fp8_kernel(const uint8_t* __restrict__ W, long long ldw, int tiled, const uint8_t* __restrict__ S,
                                   long long lds, int N, int K, uint16_t* __restrict__ out, long long ldo) {
    const long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int kq = K >> 4;
    if (q >= (long long)N * kq) return;
    const int n = (int)(q / kq), k16 = (int)(q % kq);
    const uint8_t* src;
    if (tiled) {
        const int c = k16 >> 2, jj = k16 & 3;
        src = W + (((long long)(n >> 4) * (K >> 6) + c) * 64 + jj * 16 + (n & 15)) * 16;
    } else {
        src = W + (long long)n * ldw + (long long)k16 * 16;
    }
    const v4i w = *(const v4i*)src;
    const uint32_t b = S[(long long)(n >> 5) * lds + (k16 >> 1)];
    uint32_t o[8];
    const uint32_t words[4] = {(uint32_t)w.x, (uint32_t)w.y, (uint32_t)w.z, (uint32_t)w.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t c0 = (words[i >> 1] >> (16 * (i & 1))) & 0xFFu, c1 = (words[i >> 1] >> (16 * (i & 1) + 8)) & 0xFFu;
        const uint32_t lo = f32_to_bf16_bits(__uint_as_float(e4m3_e8m0_f32_bits(c0, b)));
        const uint32_t hi = f32_to_bf16_bits(__uint_as_float(e4m3_e8m0_f32_bits(c1, b)));
        o[i] = lo | (hi << 16);
    }
    v4i* dst = (v4i*)(out + (long long)n * ldo + (long long)k16 * 16);
    dst[0] = v4i{(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
    dst[1] = v4i{(int)o[4], (int)o[5], (int)o[6], (int)o[7]};
}

// ------------------------------------------------------------------------------------------ entry points
template <int MT, int PF, int RB = 1>
static void fp8_launch_pf(const Fp8Args& a, int tiled, bool wide, hipStream_t st) {
    const dim3 grid(((a.N + 15) / 16 + RB - 1) / RB);
    if (wide) {
        if (tiled) fp8_gemm_kernel<16, PF, MT, 1, RB><<<grid, 1024, 0, st>>>(a);
        else fp8_gemm_kernel<16, PF, MT, 0, RB><<<grid, 1024, 0, st>>>(a);
    } else {
        if (tiled) fp8_gemm_kernel<8, PF, MT, 1, RB><<<grid, 512, 0, st>>>(a);
        else fp8_gemm_kernel<8, PF, MT, 0, RB><<<grid, 512, 0, st>>>(a);
    }
}

template <int MT>
static void fp8_launch(const Fp8Args& a, int tiled, hipStream_t st) {
    const int nb = (a.N + 15) / 16;
    // few row blocks: 16 waves per workgroup so the K split still fills the CUs (not for 4 token tiles, whose
    // registers do not fit 16 waves per CU)
    const bool wide = MT <= 2 && nb < 256 && a.nk >= 64;
    // >= 256 row blocks: two row blocks per 8-wave workgroup (every activation load feeds two weight tiles); one token
    // tile: 4 tiles in flight per wave, 3 when a wave has fewer than 4 chunks; two: 3; four: 2. Measured (median of 50
    // graph replays, against one row block per workgroup): 16 / 8 rows 5120 x 8192 20.4 -> 14.4 / 14.9 -> 12.0 us,
    // 4608 x 5120 14.3 -> 10.6 / 10.7 -> 9.0, 32768 x 1280 15.6 -> 12.1 / 11.4 -> 10.5, 5120 x 2304 7.6 -> 6.5 / 6.1 ->
    // 6.0; 32 / 64 rows 5120 x 8192 33.9 -> 21.0 / 63.7 -> 36.4, 32768 x 1280 27.8 -> 20.1 / 52.3 -> 38.4. 16-wave
    // workgroups were level or slower, four row blocks per workgroup slower (5120 x 8192 at 16 rows: 19.8), and fewer
    // row blocks (1280 x 5120: 40 workgroups) slower (8.2 -> 9.9 at 16 rows), so they keep one block each
    if (nb >= 256 && (a.gc == 0 || a.gc % 32 == 0)) {
        if (MT == 1 && a.nk < 32) fp8_launch_pf<1, 3, 2>(a, tiled, false, st);
        else fp8_launch_pf<MT, MT == 1 ? 4 : MT == 2 ? 3 : 2, 2>(a, tiled, false, st);
        return;
    }
    // one row block per workgroup, <= 128 VGPRs: two 8-wave workgroups per CU. One token tile: 6 tiles in flight per
    // wave, 3 when a wave has fewer than 6 chunks (measured at 16 / 8 rows: 32768 x 1280 17.9 -> 15.1 / 14.8 -> 11.0 us;
    // the other reference shapes within 1 %, and 2 / 4 / 8 in flight no better)
    if (MT == 1 && a.nk < 6 * (wide ? 16 : 8)) fp8_launch_pf<MT, 3>(a, tiled, wide, st);
    else fp8_launch_pf<MT, MT == 1 ? 6 : MT == 2 ? 4 : 2>(a, tiled, wide, st);
}

extern "C" int dsv41_fp8_gemm(const uint8_t* W, long long ldw, int tiled, const uint8_t* S, long long lds, int N, int K,
                              const uint16_t* x, long long ldx, int M, int group_cols, float* out, long long ldo,
                              uint16_t* outb, long long ldob, void* stream) {
    if (!W || !S || !x || (!out && !outb) || N <= 0 || K <= 0 || (K & 63) || M < 1 || M > 64) return DSV41_EINVAL;
    if (tiled ? ((N & 15) || ldw != K) : ldw < K) return DSV41_EINVAL;
    if (lds < K / 32 || ldx < K || (out && ldo < N) || (outb && ldob < N)) return DSV41_EINVAL;
    if (group_cols < 0 || (group_cols && ((group_cols & 15) || N % group_cols))) return DSV41_EINVAL;
    const long long G = group_cols ? N / group_cols : 1;
    Fp8Args a{W, ldw, S, lds, N, K, K / 64, x, ldx, ldx * G, M, group_cols, out, ldo, outb, ldob};
    hipStream_t st = (hipStream_t)stream;
    // up to 4 tokens whose activations fit 64 KiB of LDS per workgroup: the LDS-staged kernel. Launch shapes, measured
    // at one token over resident copies larger than the 256 MB last-level cache (median of 50 graph replays):
    //  * >= 256 row blocks: 4 waves per workgroup, 4 weight tiles in flight per wave (5120 x 8192: 9.5 us; 12 in flight
    //    10.9, 24 12.1, 8 waves 10.7-11.0, 16 waves 12.2-13.1); rows of <= 24 chunks (K <= 1536) 2 waves, each with
    //    more of the row (32768 x 1280: 9.2 us against 10.1 with 4 waves);
    //  * fewer row blocks: 4 waves with 10 tiles in flight (1280 x 5120: 5.0 us against 5.9 with 16 waves).
    // Deeper prefetch was slower for every shape with more row blocks than CUs.
    const int nb = (N + 15) / 16;
    const int wpg = nb >= 256 && a.nk <= 24 ? 2 : 4;
    const int cpw = (a.nk + wpg - 1) / wpg;
    const long long lds_bytes = (long long)wpg * fp8_lds_region(M, cpw);
    // every wave owns >= 1 chunk; activation pieces and scale bytes fit the per-lane staging registers
    if (M <= 4 && a.nk >= wpg && M * cpw <= 64 && 2 * cpw <= 128 && lds_bytes <= 65536) {
        const dim3 grid(nb);
        if (wpg == 2) {
            if (tiled) fp8_gemv_lds_kernel<2, 4, 1><<<grid, 128, lds_bytes, st>>>(a, cpw);
            else fp8_gemv_lds_kernel<2, 4, 0><<<grid, 128, lds_bytes, st>>>(a, cpw);
        } else if (nb >= 256) {
            if (tiled) fp8_gemv_lds_kernel<4, 4, 1><<<grid, 256, lds_bytes, st>>>(a, cpw);
            else fp8_gemv_lds_kernel<4, 4, 0><<<grid, 256, lds_bytes, st>>>(a, cpw);
        } else {
            if (tiled) fp8_gemv_lds_kernel<4, 10, 1><<<grid, 256, lds_bytes, st>>>(a, cpw);
            else fp8_gemv_lds_kernel<4, 10, 0><<<grid, 256, lds_bytes, st>>>(a, cpw);
        }
        return (int)hipGetLastError();
    }
    // more tokens x chunks than 4 waves can stage: 8 waves (16 for few row blocks with long rows), 12 tiles in flight
    const int wpg2 = nb < 256 && a.nk >= 64 ? 16 : 8, cpw2 = (a.nk + wpg2 - 1) / wpg2;
    const long long lds2 = (long long)wpg2 * fp8_lds_region(M, cpw2);
    if (M <= 4 && a.nk >= wpg2 && M * cpw2 <= 64 && 2 * cpw2 <= 128 && lds2 <= 65536) {
        const dim3 grid(nb);
        if (wpg2 == 16) {
            if (tiled) fp8_gemv_lds_kernel<16, 12, 1><<<grid, 1024, lds2, st>>>(a, cpw2);
            else fp8_gemv_lds_kernel<16, 12, 0><<<grid, 1024, lds2, st>>>(a, cpw2);
        } else {
            if (tiled) fp8_gemv_lds_kernel<8, 12, 1><<<grid, 512, lds2, st>>>(a, cpw2);
            else fp8_gemv_lds_kernel<8, 12, 0><<<grid, 512, lds2, st>>>(a, cpw2);
        }
        return (int)hipGetLastError();
    }
    if (M <= 16) fp8_launch<1>(a, tiled, st);
    else if (M <= 32) fp8_launch<2>(a, tiled, st);
    else fp8_launch<4>(a, tiled, st);
    return (int)hipGetLastError();
}

extern "C" int dsv41_dequant_fp8(const uint8_t* W, long long ldw, int tiled, const uint8_t* S, long long lds, int N, int K,
                                 uint16_t* out, long long ldo, void* stream) {
    if (!W || !S || !out || N <= 0 || K <= 0 || (K & 15) || ldo < K || lds < (K + 31) / 32) return DSV41_EINVAL;
    if (tiled ? ((N & 15) || (K & 63) || ldw != K) : ldw < K) return DSV41_EINVAL;
    const long long n16 = (long long)N * (K / 16);
    dequant_fp8_kernel<<<(unsigned)((n16 + 255) / 256), 256, 0, (hipStream_t)stream>>>(W, ldw, tiled, S, lds, N, K, out, ldo);
    return (int)hipGetLastError();
}
