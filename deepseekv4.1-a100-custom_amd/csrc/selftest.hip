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

// MFMA issue-rate probe: every lane runs `iters` rounds of 8 independent block-scaled 16x16x128 MFMAs on registers
// (no memory traffic), so the launch time measures the matrix pipes' sustained rate for one operand-format mix.
// mode 0: FP4 weights x FP8 activations (the expert kernels' mix), 1: FP8 x FP8, 2: FP4 x FP4.
template <int AF, int BF>
__global__ void __launch_bounds__(256) selftest_mfma_rate_kernel(int iters, float* out, int seed) {
    v8i a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (seed * ((int)threadIdx.x + i)) | 0x11111111;
        b[i] = seed ^ ((int)threadIdx.x * 7 + i);
    }
    if (AF == 4) { a[4] = a[5] = a[6] = a[7] = 0; }   // FP4 operands use the low 4 dwords
    if (BF == 4) { b[4] = b[5] = b[6] = b[7] = 0; }
    v4f c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c[j], AF, BF, 0, 127, 0, 127);
    }
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    if (sum == 1234.5f) out[0] = sum;   // keeps the MFMAs live; never true for these operands' finite sums in practice
}

extern "C" int dsv41_selftest_mfma_rate(int mode, int blocks, int iters, float* out, void* stream) {
    if (!out || blocks < 1 || iters < 1 || mode < 0 || mode > 2) return DSV41_EINVAL;
    hipStream_t st = (hipStream_t)stream;
    if (mode == 0) selftest_mfma_rate_kernel<4, 0><<<blocks, 256, 0, st>>>(iters, out, 3);
    else if (mode == 1) selftest_mfma_rate_kernel<0, 0><<<blocks, 256, 0, st>>>(iters, out, 3);
    else selftest_mfma_rate_kernel<4, 4><<<blocks, 256, 0, st>>>(iters, out, 3);
    return (int)hipGetLastError();
}

// HBM stream-rate probe: `blocks` workgroups of WAVES waves read `tiles` 1 KiB tiles of src once. Workgroup b takes the
// contiguous tiles [tiles b / blocks, tiles (b + 1) / blocks); its waves interleave over them (wave j: tile j, j + WAVES,
// ...), 8 tiles in flight per wave, with the decode kernels' nontemporal buffer loads. Every wave of a workgroup runs the
// same number of iterations (a last iteration past the workgroup's tiles reads zeros through the descriptor bound), so
// SYNC = 1 can add a workgroup barrier after every second tile, as the prefill kernels synchronise each k-step. out is
// written only if the bytes XOR to one particular word (keeps the loads live).
template <int WAVES, int SYNC>
__global__ void __launch_bounds__(WAVES * 64) selftest_stream_kernel(const uint8_t* src, long long tiles, unsigned* out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const long long t0 = tiles * blockIdx.x / gridDim.x, t1 = tiles * (blockIdx.x + 1) / gridDim.x;
    const int n = (int)((t1 - t0 + WAVES - 1) / WAVES);
    const __amdgpu_buffer_rsrc_t r = buffer_rsrc(src + t0 * 1024, (uint32_t)((t1 - t0) * 1024));
    const uint32_t voff = (uint32_t)(wave * 1024 + lane * 16);
    v4i A[8];
    unsigned x = 0;
    int used = 0;
    pipelined<8>(n, [&](int slot, int i) { A[slot] = buffer_load_tile(r, voff, (uint32_t)i * (WAVES * 1024u)); },
                 [&](int slot) {
                     x ^= (unsigned)(A[slot].x ^ A[slot].y ^ A[slot].z ^ A[slot].w);
                     if (SYNC && (++used & 1) == 0) __builtin_amdgcn_s_barrier();
                 });
    if (x == 0x9E3779B9u) out[0] = x;   // keeps the loads live (a store only if the bytes happen to XOR to this word)
}

extern "C" int dsv41_selftest_stream(const uint8_t* src, long long tiles, int blocks, int waves, int sync, unsigned* out, void* stream) {
    if (!src || !out || tiles < 1 || blocks < 1 || (waves != 4 && waves != 8) || sync < 0 || sync > 1) return DSV41_EINVAL;
    if ((tiles + blocks - 1) / blocks * 1024 > 0xFFFFFFFFll) return DSV41_EINVAL;   // one workgroup's bytes: 32-bit offsets
    hipStream_t st = (hipStream_t)stream;
    if (waves == 8) {
        if (sync) selftest_stream_kernel<8, 1><<<blocks, 512, 0, st>>>(src, tiles, out);
        else selftest_stream_kernel<8, 0><<<blocks, 512, 0, st>>>(src, tiles, out);
    } else {
        if (sync) selftest_stream_kernel<4, 1><<<blocks, 256, 0, st>>>(src, tiles, out);
        else selftest_stream_kernel<4, 0><<<blocks, 256, 0, st>>>(src, tiles, out);
    }
    return (int)hipGetLastError();
}

// FP8 conversion check: for input i, the code of v[i] at scale 2^e[i] by bit arithmetic (fq8_code_sw) and by the
// hardware conversion (fq8_code2_hw, both halves of the pair), and the decoded value of the software code both ways.
// out[5 i ..]: sw code, hw code (low byte of the pair), hw code (high byte), bits of the sw decode, bits of the hw decode.
__global__ void __launch_bounds__(256) selftest_fp8_cvt_kernel(const float* v, const int* e, int n, uint32_t* out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float x = v[i];
    const int ex = e[i];
    const uint32_t sw = fq8_code_sw(x, ex);
    const uint32_t hw = fq8_code2_hw(x, -x, ex);
    uint32_t* o = out + 5ll * i;
    o[0] = sw;
    o[1] = hw & 0xFFu;
    o[2] = (fq8_code4_hw(0.f, 0.f, -x, x, ex) >> 24) & 0xFFu;   // the second pair's high byte: x again
    o[3] = __float_as_uint(fq8_value(sw, ex));
    o[4] = __float_as_uint(fq8_value_hw<0>(sw, ex));
    (void)hw;
}

extern "C" int dsv41_selftest_fp8_cvt(const float* v, const int* e, int n, uint32_t* out, void* stream) {
    if (!v || !e || !out || n < 0) return DSV41_EINVAL;
    if (n == 0) return 0;
    selftest_fp8_cvt_kernel<<<(unsigned)((n + 255) / 256), 256, 0, (hipStream_t)stream>>>(v, e, n, out);
    return (int)hipGetLastError();
}
