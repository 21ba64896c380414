// Router logits of the next MoE layer with the layer-to-layer step fused in, for M <= 16 token rows:
//   r  = bf16(x + y)                                  (y NULL: r = x)
//   xn = bf16(r * rsqrt(mean(r^2) + eps) * w)         (fused.rmsnorm, fused.py:92-110; w NULL = ones)
//   logits[t][e] = sum_k xn[t][k] * G[e][k]           (the router GEMV, model.py:391-392; decode.py:357)
// The GEMV is split along K into KS = H / 1024 parts so the 5.5 MB of router weights stream through
// (E / 16) x KS workgroups: part[ks][t][e] holds the sum over k in [1024 ks, 1024 ks + 1024). The gate adds the KS
// parts in ascending order (gate_row_wave's nparts), so the logits are deterministic. The workgroups also
// write xn and xq = fake_quant_fp8(xn) (quant.py:34-54) for the experts and the next step: the workgroups of
// row block 0 each write their own k range.
// Each workgroup recomputes the rms statistics of all M rows (M x 28 KB of L2 reads, one round trip per row)
// rather than waiting on another launch; its 16 x 1024 weight tile is in flight meanwhile, and the threads that hold
// its own k range of r keep it in LDS, so nothing is loaded twice.
#include "common.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define RT_THREADS 512
#define RT_KC 1024     // k per workgroup: 8 waves x 128
#define RT_MAXM 16

struct RouterArgs {
    const uint16_t* x; long long ldx;
    const uint16_t* y; long long ldy;
    const uint16_t* w; float eps;
    const uint16_t* G; long long ldg;   // bf16 [E][ldg]
    int E, H, M;
    float* part;                        // fp32 [KS][M][E]
    uint16_t* xn; long long ldn;        // bf16 [M][H] (written by the workgroups of row block 0)
    uint16_t* xq; long long ldq;
};

__device__ __forceinline__ void unpack8(const v4i v, float* f) {
    const uint32_t w[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf16_to_f32(w[j] & 0xFFFFu);
        f[2 * j + 1] = bf16_to_f32(w[j] >> 16);
    }
}

// The x and y vectors of a thread's two 8-element pieces of row t (pieces tid and tid + 512, clamped to the row;
// y NULL: x again, ignored), all four loads issued together.
struct RowRaw { v4i x[2], y[2]; };
__device__ __forceinline__ RowRaw load_row_raw(const RouterArgs& a, int t, int tid, int nvec) {
    const uint16_t* yb = a.y ? a.y : a.x;
    const long long ly = a.y ? a.ldy : a.ldx;
    RowRaw r;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int k = min(tid + u * RT_THREADS, nvec - 1) * 8;
        r.x[u] = *(const v4i*)(a.x + (long long)t * a.ldx + k);
        r.y[u] = *(const v4i*)(yb + (long long)t * ly + k);
    }
    return r;
}

// Row t's share of this thread: r = bf16(x + y) (y NULL: r = x) of its two pieces; returns their sum of squares
// (pieces past the row weighted 0) and keeps the pieces of this workgroup's k range in s_r.
__device__ __forceinline__ float row_sumsq(const RouterArgs& a, const RowRaw& raw, int t, int tid, int nvec, int ks,
                                           float (*s_r)[RT_KC]) {
    const int nkv = RT_KC / 8;
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        float f[8], g[8];
        unpack8(raw.x[u], f);
        unpack8(raw.y[u], g);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = a.y ? bf16_round(f[j] + g[j]) : f[j];
        const float m = tid + u * RT_THREADS < nvec ? 1.f : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) ss += m * f[j] * f[j];
        const int v = tid + u * RT_THREADS - ks * nkv;
        if (v >= 0 && v < nkv) {
            *(v4f*)&s_r[t][v * 8] = v4f{f[0], f[1], f[2], f[3]};
            *(v4f*)&s_r[t][v * 8 + 4] = v4f{f[4], f[5], f[6], f[7]};
        }
    }
    return ss;
}

__global__ void __launch_bounds__(RT_THREADS) router_norm_kernel(const RouterArgs a) {
    __shared__ float s_ss[RT_THREADS / 64][RT_MAXM];
    __shared__ __align__(16) uint16_t s_xn[RT_MAXM][RT_KC + 8];
    __shared__ __align__(16) float s_r[RT_MAXM][RT_KC];   // this workgroup's k range of r
    __shared__ __align__(16) float s_w[RT_KC];            // and of the norm weight
    __shared__ v4f s_acc[RT_THREADS / 64][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = blockIdx.x, ks = blockIdx.y;
    const int M = a.M, H = a.H, nvec = H >> 3;
    const int col = lane & 15, kg = lane >> 4;
    const int k0 = ks * RT_KC + wave * 128;

    // Row 0 of r and the norm weight of this workgroup's k range (thread tid < 128 holds 8 values; NULL: ones) are
    // L2 hits; their sum of squares is taken before the weight tiles go out. Issued behind the tiles (which come
    // from HBM, and loads return in issue order) they kept the whole rms chain waiting on them: 5.8 -> 4.8 us.
    const int nkv = RT_KC / 8;
    const RowRaw row0 = load_row_raw(a, 0, tid, nvec);
    const v4i wraw = *(const v4i*)((a.w ? a.w : a.x) + ks * RT_KC + min(tid, nkv - 1) * 8);
    float ss0 = row_sumsq(a, row0, 0, tid, nvec, ks, s_r);
    __builtin_amdgcn_sched_barrier(0);
    // this wave's weight tile (16 rows x 128 k): 4 loads of 16 B per lane
    v4i A[4];
    const uint16_t* gp = a.G + (long long)(rb * 16 + col) * a.ldg + k0 + kg * 8;
#pragma unroll
    for (int i = 0; i < 4; ++i) A[i] = __builtin_nontemporal_load((const v4i*)(gp + i * 32));
    __builtin_amdgcn_sched_barrier(0);

    // ---- sum of squares of r per row (a thread owns pieces tid and tid + 512: H <= 8192), one round trip per row
    for (int t = 0; t < M; ++t) {
        const float ss = wave_reduce_sum(t == 0 ? ss0 : row_sumsq(a, load_row_raw(a, t, tid, nvec), t, tid, nvec, ks, s_r));
        if (lane == 0) s_ss[wave][t] = ss;
    }
    if (tid < nkv) {
        float wv[8];
        unpack8(wraw, wv);
#pragma unroll
        for (int j = 0; j < 8; ++j) wv[j] = a.w ? wv[j] : 1.f;
        *(v4f*)&s_w[tid * 8] = v4f{wv[0], wv[1], wv[2], wv[3]};
        *(v4f*)&s_w[tid * 8 + 4] = v4f{wv[4], wv[5], wv[6], wv[7]};
    }
    __syncthreads();

    // ---- xn of this workgroup's k range into LDS; workgroups of row block 0 also write xn and xq there. Each
    // thread sums its row's eight wave partials itself (same order everywhere), so no further barrier is needed.
    for (int i = tid; i < M * nkv; i += RT_THREADS) {
        const int t = i / nkv, v = i - t * nkv;
        const int k = ks * RT_KC + v * 8;
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < RT_THREADS / 64; ++w) tot += s_ss[w][t];
        const float inv = 1.0f / sqrtf(tot / (float)H + a.eps);
        float n[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) n[j] = bf16_round(s_r[t][v * 8 + j] * inv * s_w[v * 8 + j]);
        uint32_t on[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) on[j] = f32_to_bf16_bits(n[2 * j]) | (f32_to_bf16_bits(n[2 * j + 1]) << 16);
        const v4i ov = v4i{(int)on[0], (int)on[1], (int)on[2], (int)on[3]};
        *(v4i*)&s_xn[t][v * 8] = ov;
        if (rb == 0) {
            // four consecutive threads hold one FP8 group (the range and the row are multiples of 32 elements)
            float amax = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(n[j]));
            amax = fmaxf(amax, __shfl_xor(amax, 1, 4));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 4));
            const int e = fq8_exponent(amax);
            uint32_t oq[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                oq[j] = f32_to_bf16_bits(fq8_value(fq8_code(n[2 * j], e), e)) | (f32_to_bf16_bits(fq8_value(fq8_code(n[2 * j + 1], e), e)) << 16);
            *(v4i*)(a.xn + (long long)t * a.ldn + k) = ov;
            *(v4i*)(a.xq + (long long)t * a.ldq + k) = v4i{(int)oq[0], (int)oq[1], (int)oq[2], (int)oq[3]};
        }
    }
    __syncthreads();

    // ---- 4 MFMAs per wave (B column = token; columns past M read row 0 and are not stored)
    const int brow = col < M ? col : 0;
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const v4i b = *(const v4i*)&s_xn[brow][wave * 128 + i * 32 + kg * 8];
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, A[i]), __builtin_bit_cast(v8bf, b), acc, 0, 0, 0);
    }
    s_acc[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && col < M) {
        v4f sum = s_acc[0][lane];
#pragma unroll
        for (int w = 1; w < RT_THREADS / 64; ++w) sum += s_acc[w][lane];
        // lane l holds D[4 (l / 16) + i][l % 16]: rows = experts, column = token
        float* o = a.part + ((long long)ks * M + col) * a.E + rb * 16 + 4 * kg;
        o[0] = sum.x; o[1] = sum.y; o[2] = sum.z; o[3] = sum.w;
    }
}

extern "C" int dsv41_router_logits(const uint16_t* x, long long ldx, const uint16_t* y, long long ldy, const uint16_t* w, float eps,
                                   const uint16_t* G, long long ldg, int E, int H, int M, float* part, uint16_t* xn, long long ldn,
                                   uint16_t* xq, long long ldq, void* stream) {
    if (!x || !G || !part || !xn || !xq || M < 1 || M > RT_MAXM || E <= 0 || (E & 15) || H <= 0 || (H % RT_KC) || H > 2 * RT_THREADS * 8 ||
        ldg < H || ldx < H ||
        ldn < H || ldq < H || (y && ldy < H) || ((ldx | ldn | ldq | ldg | (y ? ldy : 0)) & 7) || !(eps >= 0.f) ||
        ((((uintptr_t)x) | ((uintptr_t)y) | ((uintptr_t)w) | ((uintptr_t)G) | ((uintptr_t)xn) | ((uintptr_t)xq)) & 15))
        return DSV41_EINVAL;
    RouterArgs a{x, ldx, y, ldy, w, eps, G, ldg, E, H, M, part, xn, ldn, xq, ldq};
    router_norm_kernel<<<dim3(E / 16, H / RT_KC), RT_THREADS, 0, (hipStream_t)stream>>>(a);
    return (int)hipGetLastError();
}

// ------------------------------------------------------------------------------------------ fp32 router weights
// Router logits with fp32 router weights (model.MoE.gate: F.linear(x.float(), gate_w) with gate_w fp32, model.py:368,
// 392), for M <= 16 bf16 rows, split along K like the kernel above: part[ks][t][e] = sum over k in [1024 ks, +1024)
// of x[t][k] * G[e][k]. fp32 MFMA 16x16x4: in one product lane l holds row e0 + l % 16 and token l % 16 at k-group
// g = l / 16. Each lane loads 16 bytes (4 consecutive k) of its row per 16-k block and uses them in 4 products
// (product i takes k = 16 j + 4 g + i), with the matching activations from LDS, so every weight load is a full
// 16-byte vector and each wave-load covers 16 rows x 64 contiguous bytes.
#define RF_THREADS 256
__global__ void __launch_bounds__(RF_THREADS) router_f32w_kernel(const uint16_t* __restrict__ x, long long ldx, const float* __restrict__ G,
                                                                 long long ldg, int E, int M, float* __restrict__ part) {
    __shared__ __align__(16) uint16_t s_x[RT_MAXM][RT_KC + 8];   // this workgroup's k range of the M rows, bf16
    __shared__ v4f s_acc[RF_THREADS / 64][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = blockIdx.x, ks = blockIdx.y;
    const int k0 = ks * RT_KC;
    const int col = lane & 15, kg = lane >> 4;
    // stage the activations first (16 bytes per thread per step; rows past M are not read): they are L2 hits, and
    // behind the weight loads they would return only after them (loads return in issue order)
    for (int i = tid; i < M * (RT_KC / 8); i += RF_THREADS) {
        const int t = i / (RT_KC / 8), v = i - t * (RT_KC / 8);
        *(v4i*)&s_x[t][v * 8] = *(const v4i*)(x + (long long)t * ldx + k0 + v * 8);
    }
    __builtin_amdgcn_sched_barrier(0);
    // the wave's 16 blocks of 16 k: all 16 weight loads in flight at once
    const int kw = k0 + wave * (RT_KC / (RF_THREADS / 64));
    // rows past E (the last block when E % 16 != 0) read row E - 1; their outputs are not stored
    const float* wr = G + (long long)min(rb * 16 + col, E - 1) * ldg + kw + 4 * kg;
    v4f A[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) A[j] = __builtin_nontemporal_load((const v4f*)(wr + 16 * j));
    __syncthreads();
    const uint16_t* xr = &s_x[col < M ? col : 0][wave * (RT_KC / (RF_THREADS / 64)) + 4 * kg];
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint2 xb = *(const uint2*)(xr + 16 * j);
        const float b[4] = {bf16_to_f32(xb.x & 0xFFFFu), bf16_to_f32(xb.x >> 16), bf16_to_f32(xb.y & 0xFFFFu), bf16_to_f32(xb.y >> 16)};
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[j].x, b[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[j].y, b[1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[j].z, b[2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[j].w, b[3], acc, 0, 0, 0);
    }
    s_acc[wave][lane] = acc;
    __syncthreads();
    if (wave == 0 && col < M) {
        v4f sum = s_acc[0][lane];
#pragma unroll
        for (int w = 1; w < RF_THREADS / 64; ++w) sum += s_acc[w][lane];
        // lane l holds D[4 (l / 16) + i][l % 16]: rows = experts, column = token
        float* o = part + ((long long)ks * M + col) * E + rb * 16 + 4 * kg;
        const float v[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (rb * 16 + 4 * kg + i < E) o[i] = v[i];
    }
}

extern "C" int dsv41_router_logits_f32w(const uint16_t* x, long long ldx, const float* G, long long ldg, int E, int H, int M, float* part,
                                        void* stream) {
    if (!x || !G || !part || M < 1 || M > RT_MAXM || E <= 0 || H <= 0 || (H % RT_KC) || ldx < H || ldg < H || (ldx & 7) ||
        (ldg & 3) || (((uintptr_t)x) & 15) || (((uintptr_t)G) & 15))
        return DSV41_EINVAL;
    router_f32w_kernel<<<dim3((E + 15) / 16, H / RT_KC), RF_THREADS, 0, (hipStream_t)stream>>>(x, ldx, G, ldg, E, M, part);
    return (int)hipGetLastError();
}
