// C ABI of the host (CPU) MoE expert library, libdsv41_cpu.so (deepseekv4.1-a100-custom_amd/cpu/host_moe.cpp).
//
// The entry points carry the names, argument order and meaning of the reference CPU library that
// dsv41/cpumoe.py binds with ctypes (cpumoe.py:24-50; dsv41/cpu/moe_cpu.cpp), so the reference's HostExperts
// can load this library instead of its own build. Layouts of the host buffers (row-major, per expert):
//   w13 [E][2*inter][dim/2] u8 (gate rows then up rows, low nibble = even k), s13 [E][2*inter][dim/32] E8M0,
//   w2  [E][dim][inter/2]   u8,                                            s2  [E][dim][inter/32]   E8M0.
// Activations are bf16 bit patterns (uint16_t), outputs fp32. Entry points that return int return 0 on success,
// -1 for more than 16 experts (as moe_cpu.cpp:550), -2 for invalid arguments (shape rules below), -3 when the
// library could not allocate its workspace. Calls are serialised inside the library (one at a time).
// Shape rules: int8 mode (the default) needs K % 128 == 0 for every GEMV (dim for stage 1, inter for stage 3);
// exact mode needs K % 32 == 0.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Worker threads pinned to CPUs 0..threads-1, cores_per_node consecutive workers per NUMA node
// (moe_cpu.cpp:41-46).
void cpumoe_init(int threads, int cores_per_node);

// Worker threads pinned to cpus[0..n-1] (node 0's CPUs first); returns the number of workers started
// (moe_cpu.cpp:48-62, which returns the OpenMP team size).
int cpumoe_init_list(const int* cpus, int n, int cores_per_node);

// No counterpart in the reference: how many workers could pin themselves to their CPU (for diagnostics).
int cpumoe_threads_pinned(void);

// Anonymous mapping with transparent huge pages unless DSV41_NO_THP is set (moe_cpu.cpp:64-71).
void* cpumoe_alloc(size_t bytes);

// No counterpart in the reference (its buffers live until exit): unmaps a cpumoe_alloc mapping.
int cpumoe_free(void* p, size_t bytes);

// MPOL_BIND each node's row range of an [E][N][row_bytes] buffer to that node; returns the number of
// ranges that failed (moe_cpu.cpp:78-91).
int cpumoe_bind_rows(uint8_t* base, int E, int N, int row_bytes);

// Fraction of sampled 2 MiB pages of each node's row range that live on that node, -1 when nothing could be
// sampled (moe_cpu.cpp:102-116).
double cpumoe_local_fraction(const uint8_t* base, int E, int N, int row_bytes);

// Copy an [N][row_bytes] matrix, each node's threads first-touching the rows that node reads
// (moe_cpu.cpp:122-136).
void cpumoe_load_rows(uint8_t* dst, const uint8_t* src, int N, int row_bytes);

// Best-of-iters read bandwidth in GB/s over p[0..bytes): node_sel -1 = every node reads its share,
// k = only node k reads its share (moe_cpu.cpp:139-165).
double cpumoe_bw_test(const uint8_t* p, size_t bytes, int iters, int node_sel);

// Largest row chunk handed out at once in stage 1 / stage 3 (moe_cpu.cpp:383; ch3 <= 256).
void cpumoe_set_chunks(int ch1, int ch3);

// 0: exact mode (fp32 dequantised weights); any other value: int8 mode (moe_cpu.cpp:384, modes 1 and 2).
void cpumoe_set_int8(int on);

// No counterpart in the reference (its distance is the compile-time PF_DIST, moe_cpu.cpp:233-235): software
// prefetch distance along a weight row in bytes, 0 = off.
void cpumoe_set_prefetch(int bytes);

// One token through E <= 16 experts: out[dim] = sum_e h_e . w2_e with h_e = fq8(bf16(wts[e] * silu(g) * u)),
// (g, u) = x . w13_e (clamped at `limit` when limit > 0). gu [E][2*inter] fp32 and h [E][inter] bf16 are
// caller scratch and hold the stage-1 and stage-2 results on return (moe_cpu.cpp:386-503).
int cpumoe_forward(const uint8_t* const* w13, const uint8_t* const* s13, const uint8_t* const* w2, const uint8_t* const* s2, int E,
                   const uint16_t* x, const float* wts, float* out, int K, int inter, int dim, float limit, float* gu, uint16_t* h);

// cpumoe_forward with expert e at base + ids[e] * stride for each of the four buffers (moe_cpu.cpp:545-553).
int cpumoe_forward_ids(const uint8_t* w13, const uint8_t* s13, const uint8_t* w2, const uint8_t* s2, size_t b13, size_t bs13, size_t b2,
                       size_t bs2, const int* ids, int E, const uint16_t* x, const float* wts, float* out, int K, int inter, int dim,
                       float limit, float* gu, uint16_t* h);

// Copy one expert (w1, w3, s1, s3, w2, s2 source rows) into slot e of the layer buffers, each node's threads
// copying the rows that node reads (moe_cpu.cpp:557-587).
void cpumoe_load_expert(uint8_t* w13, uint8_t* s13, uint8_t* w2, uint8_t* s2, int e, const uint8_t* src_w1, const uint8_t* src_w3,
                        const uint8_t* src_s1, const uint8_t* src_s3, const uint8_t* src_w2, const uint8_t* src_s2, int inter, int dim);

// Copy a whole layer (arrays of E source pointers per matrix) into the layer buffers (moe_cpu.cpp:509-541).
void cpumoe_load_layer(uint8_t* w13, uint8_t* s13, uint8_t* w2, uint8_t* s2, const uint8_t* const* sw1, const uint8_t* const* sw3,
                       const uint8_t* const* ss1, const uint8_t* const* ss3, const uint8_t* const* sw2, const uint8_t* const* ss2,
                       int E, int inter, int dim);

// One FP4 GEMV out[N] = W[N][K] . x[K] (packed E2M1 w [N][K/2], E8M0 s [N][K/32], bf16 x), in the current
// mode. The reference has no single-matrix CPU entry; its per-row kernels are dot_row_v2 / dot_row
// (moe_cpu.cpp:177-205,237-275), and the GPU twin of this GEMV is cukern.fp4_gemv_pairs with one pair.
int cpumoe_gemv(const uint8_t* w, const uint8_t* s, int N, int K, const uint16_t* x, float* out);

#ifdef __cplusplus
}
#endif
