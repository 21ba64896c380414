// Dense bf16 GEMV for M <= 16 tokens on bf16 MFMA (v_mfma_f32_16x16x32_bf16): the bf16 shared expert of the
// MoE layer (model.py:409-412, decode.py:369-371, bf16 weights as the benchmark configuration specifies) and the
// router logits x . G^T (model.py:391-392, decode.py:357).
//   out[t, n] = sum_k x[t, k] * W[n, k]    W bf16 [N][K] row-major, x bf16 [M][K]
// HBM-bound: a workgroup owns one 16-row block; its WPG waves split K, stream 16 x 64 B row pieces per MFMA
// (1 KiB per wave-load) and reduce through LDS in a fixed order.
#include "common.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

struct DenseArgs {
    const uint16_t* W; long long ldw;   // elements
    int N, K;
    const uint16_t* x; long long ldx;
    int M;
    float* out; long long ldo;          // optional fp32
    uint16_t* outb; long long ldob;     // optional bf16
};

// TILED: W in 16 x 32 tiles of 1 KiB ([N/16][K/32][16][32], ldw = K): a wave-load is one contiguous block.
template <int WPG, int PF, int TILED>
__global__ void __launch_bounds__(WPG * 64) dense_gemv_bf16_kernel(const DenseArgs a) {
    __shared__ v4f s_red[WPG][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = blockIdx.x;
    const int col = lane & 15, kb = lane >> 4;
    const int nk = a.K >> 5;                               // 32-k chunks
    const int c0 = (int)((long long)nk * wave / WPG), c1 = (int)((long long)nk * (wave + 1) / WPG);
    const uint16_t* wrow = TILED ? a.W + (long long)nb * 16 * a.ldw + col * 32 + kb * 8 + (long long)c0 * 512
                                 : a.W + ((long long)nb * 16 + col) * a.ldw + kb * 8 + (long long)c0 * 32;
    constexpr int cstep = TILED ? 512 : 32;   // elements from one 32-k chunk to the next
    const bool ok = col < a.M;
    // columns without a token read row 0 (their outputs are not stored): no divergent loads
    const uint16_t* xrow = a.x + (long long)(ok ? col : 0) * a.ldx + kb * 8 + (long long)c0 * 32;
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    v4i A[PF], B[PF];
    pipelined<PF>(c1 - c0,
        [&](int slot, int c) {
            A[slot] = __builtin_nontemporal_load((const v4i*)(wrow + (long long)c * cstep));
            B[slot] = *(const v4i*)(xrow + (long long)c * 32);
        },
        [&](int slot) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, A[slot]), __builtin_bit_cast(v8bf, B[slot]), acc, 0, 0, 0);
        });
    s_red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    v4f sum = s_red[0][lane];
#pragma unroll
    for (int w = 1; w < WPG; ++w) sum += s_red[w][lane];
    if (!ok) return;
    const int row0 = nb * 16 + 4 * kb;
    const float v[4] = {sum.x, sum.y, sum.z, sum.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (a.out) a.out[(long long)col * a.ldo + row0 + i] = v[i];
        if (a.outb) a.outb[(long long)col * a.ldob + row0 + i] = (uint16_t)f32_to_bf16_bits(v[i]);
    }
}

extern "C" int dsv41_dense_gemv_bf16(const uint16_t* W, long long ldw, int tiled, int N, int K, const uint16_t* x, long long ldx, int M,
                                     float* out, long long ldo, uint16_t* outb, long long ldob, void* stream) {
    if (!W || !x || (!out && !outb) || N <= 0 || (N & 15) || K <= 0 || (K & 31) || M < 1 || M > 16 || ldw < K || ldx < K || (tiled && ldw != K))
        return DSV41_EINVAL;
    if ((out && ldo < N) || (outb && ldob < N)) return DSV41_EINVAL;
    DenseArgs a{W, ldw, N, K, x, ldx, M, out, ldo, outb, ldob};
    hipStream_t st = (hipStream_t)stream;
    if (tiled) {
        if (K >= 4096) dense_gemv_bf16_kernel<8, 8, 1><<<N / 16, 512, 0, st>>>(a);
        else dense_gemv_bf16_kernel<4, 8, 1><<<N / 16, 256, 0, st>>>(a);
    } else {
        if (K >= 4096) dense_gemv_bf16_kernel<8, 8, 0><<<N / 16, 512, 0, st>>>(a);
        else dense_gemv_bf16_kernel<4, 8, 0><<<N / 16, 256, 0, st>>>(a);
    }
    return (int)hipGetLastError();
}
