// Decode MoE experts (routing + up projection + SwiGLU + down projection + combine) for callers that cannot
// allocate device memory (code under HIP graph capture that must not call hipMalloc, tight serving loops,
// harnesses that forbid allocation). The two decode launches of dsv41_moe_decode_up / dsv41_moe_down_sum run with
// their intermediates (the FP8 h rows, their E8M0 bytes and the bucketing tables) in a file-scope device array
// instead of caller-provided buffers.
//
// The array is one per GPU (each device holds its own copy, at its own address, until the process ends). Its
// address is looked up once per device with hipGetSymbolAddress, with that device current, on the entry point's
// first call there, and that pointer (never the array's host-side name) is what the launches receive. Every call
// on a GPU uses the same array and leaves its contents behind: the one region that must start at zero (the all-zero
// h row the down projection reads for tokens a group does not contain) is cleared by a fill kernel on every call.
// Calls that overlap on one GPU (other streams, other host threads) race on the array.
#include <mutex>

#include "common.h"

#define NOALLOC_SCRATCH_BYTES (2u << 20)   // 2 MiB per GPU
#define NOALLOC_MAX_DEVICES 64

static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

static uint8_t* g_scratch[NOALLOC_MAX_DEVICES];
static std::mutex g_scratch_mu;

// the device address of this GPU's array (looked up on first use), or NULL with *err set
static uint8_t* scratch_ptr(int* err) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) { *err = (int)e; return nullptr; }
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) { *err = DSV41_EINVAL; return nullptr; }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) { *err = e != hipSuccess ? (int)e : DSV41_EINVAL; return nullptr; }
        g_scratch[dev] = (uint8_t*)p;
    }
    return g_scratch[dev];
}

__global__ void __launch_bounds__(256) zero_bytes_kernel(uint8_t* __restrict__ a, int na, uint8_t* __restrict__ b, int nb) {
    for (int i = threadIdx.x; i < na; i += blockDim.x) a[i] = 0;
    for (int i = threadIdx.x; i < nb; i += blockDim.x) b[i] = 0;
}

static inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

extern "C" int dsv41_moe_experts_noalloc(const float* logits, long long ldl, int nparts, long long part_stride, const float* bias, float temp,
                                         float route_scale, int score_func, int norm, const int* eid_in, const float* wt_in, int M, int topk,
                                         int E, const uint16_t* x, long long ldx, const uint8_t* W13, long long stride_w13, const uint8_t* S13,
                                         long long stride_s13, const uint8_t* W2, long long stride_w2, const uint8_t* S2, long long stride_s2,
                                         int tiled, int H, int I, float limit, int* eid_out, float* wt_out, float* y, long long ldy,
                                         const uint16_t* ys, long long ldys, uint16_t* yb, long long ldyb, void* stream) {
    if (M < 1 || M > 16 || topk < 1 || topk > 16 || I <= 0 || (I & 127) || H <= 0 || (H & 15) || (!y && !yb)) return DSV41_EINVAL;
    // the down projection's argument checks, made here so that a rejected call launches nothing (the up projection
    // checks its own before it launches)
    if (!W2 || !S2 || stride_w2 <= 0 || stride_w2 > 0xFFFFFFFFll || stride_s2 <= 0 || stride_s2 > 0xFFFFFFFFll ||
        stride_w2 < (long long)H * (I / 2) || stride_s2 < (long long)H * (I / 32) || (y && ldy < H) || (yb && ldyb < H) || (yb && ys && ldys < H))
        return DSV41_EINVAL;
    // layout of one call: h codes [P + 1][I], h E8M0 [P + 1][I / 32] (row P all zero), then the tables
    const int P = M * topk;
    const size_t off_hs = align256((size_t)(P + 1) * I);
    const size_t off_ge = off_hs + align256((size_t)(P + 1) * (I / 32));
    const size_t off_gs = off_ge + align256((size_t)P * 4);
    const size_t off_tok = off_gs + align256((size_t)(P + 1) * 4);
    const size_t off_wt = off_tok + align256((size_t)P * 4);
    const size_t need = off_wt + align256((size_t)P * 4);
    if (need > NOALLOC_SCRATCH_BYTES) return DSV41_ENOSPACE;
    int err = 0;
    uint8_t* base = scratch_ptr(&err);
    if (!base) return err;
    uint8_t* hc = base;
    uint8_t* hs = base + off_hs;
    int* grp_expert = (int*)(base + off_ge);
    int* grp_start = (int*)(base + off_gs);
    int* tok_sorted = (int*)(base + off_tok);
    float* wt_sorted = (float*)(base + off_wt);
    int r = dsv41_moe_decode_up(logits, ldl, nparts, part_stride, bias, temp, route_scale, score_func, norm, eid_in, wt_in, M, topk, E, x, ldx,
                                W13, stride_w13, S13, stride_s13, tiled, H, I, limit, hc, I, hs, I / 32, eid_out, wt_out, grp_expert,
                                grp_start, tok_sorted, wt_sorted, nullptr, 0, 0, nullptr, 0, nullptr, 0, stream);
    if (r) return r;
    // row P, left behind by an earlier call with more pairs, holds that call's h: cleared after the up projection
    // (which writes rows < P only) and before the down projection reads it; a kernel, not a memset node, so the call
    // may be captured in a graph
    zero_bytes_kernel<<<1, 256, 0, (hipStream_t)stream>>>(hc + (size_t)P * I, I, hs + (size_t)P * (I / 32), I / 32);
    r = (int)hipGetLastError();
    if (r) return r;
    return dsv41_moe_down_sum(W2, stride_w2, S2, stride_s2, tiled, H, I, hc, I, hs, I / 32, P, grp_expert, grp_start, tok_sorted, P, M, y, ldy,
                              ys, ldys, yb, ldyb, 0, E, nullptr, 0, nullptr, 0, 0, 0.f, nullptr, 0, nullptr, nullptr, nullptr, nullptr, 0,
                              stream);
}
