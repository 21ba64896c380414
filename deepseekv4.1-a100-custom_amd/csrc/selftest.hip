// Diagnostic entry points: one wave runs one matrix instruction on caller-given operands, so a test can check
// the lane layouts the kernels rely on (which lane holds which row / column / k-block, and which scale byte
// applies where) against a CPU evaluation.
#include "common.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// a, b: [64 lanes][8 dwords]; sa, sb: [64] E8M0 bytes in bits 0..7; c: [64][4]
__global__ void __launch_bounds__(64) selftest_mfma_scale_kernel(const v8i* a, const v8i* b, const int* sa, const int* sb, v4f* c, int fmt_a, int fmt_b) {
    const int l = threadIdx.x;
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    if (fmt_a == 4 && fmt_b == 0) acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[l], b[l], acc, 4, 0, 0, sa[l], 0, sb[l]);
    else if (fmt_a == 0 && fmt_b == 0) acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[l], b[l], acc, 0, 0, 0, sa[l], 0, sb[l]);
    else if (fmt_a == 4 && fmt_b == 4) acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[l], b[l], acc, 4, 4, 0, sa[l], 0, sb[l]);
    c[l] = acc;
}

// a, b: [64 lanes][8 bf16]; c: [64][4]
__global__ void __launch_bounds__(64) selftest_mfma_bf16_kernel(const v8bf* a, const v8bf* b, v4f* c) {
    const int l = threadIdx.x;
    c[l] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[l], b[l], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
}

extern "C" int dsv41_selftest_mfma_scale(const int* a, const int* b, const int* sa, const int* sb, float* c, int fmt_a, int fmt_b, void* stream) {
    if (!a || !b || !sa || !sb || !c) return DSV41_EINVAL;
    if (!((fmt_a == 4 && fmt_b == 0) || (fmt_a == 0 && fmt_b == 0) || (fmt_a == 4 && fmt_b == 4))) return DSV41_EINVAL;
    selftest_mfma_scale_kernel<<<1, 64, 0, (hipStream_t)stream>>>((const v8i*)a, (const v8i*)b, sa, sb, (v4f*)c, fmt_a, fmt_b);
    return (int)hipGetLastError();
}

extern "C" int dsv41_selftest_mfma_bf16(const uint16_t* a, const uint16_t* b, float* c, void* stream) {
    if (!a || !b || !c) return DSV41_EINVAL;
    selftest_mfma_bf16_kernel<<<1, 64, 0, (hipStream_t)stream>>>((const v8bf*)a, (const v8bf*)b, (v4f*)c);
    return (int)hipGetLastError();
}
