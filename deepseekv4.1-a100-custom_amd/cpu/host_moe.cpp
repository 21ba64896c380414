// Host (CPU) MoE expert path: one token through up to 16 selected experts, computed straight from the packed
// E2M1 weights and E8M0 per-32 scales held in host memory. It restates the algorithm of the reference CPU
// library (dsv41/cpu/moe_cpu.cpp:386-503, driven by dsv41/cpumoe.py:123-210) behind the same C ABI (cpumoe_*):
//
//   stage 1  gu[e][n] = x . W13[e][n]                      n < 2I: the I gate rows, then the I up rows
//   stage 2  h[e][i]  = fq8(bf16(wt_e * silu(g) * u))     g = min(gate, L), u = clamp(up, -L, L) (L = 0: none),
//                                                          fq8 = FP8 E4M3 fake quantisation per 32 columns
//   stage 3  out[n]   = sum_e h[e] . W2[e][n]              experts summed in selection order
//
// Numerics, mode "int8" (the default; moe_cpu.cpp:210-228,237-275): the activation of a GEMV (x for stage 1,
// h[e] for stage 3) is re-quantised per 32 elements to symmetric int8, q = clamp(rint(v * (1 / s)), -127, 127)
// with s = amax / 127 (s = 1 for an all-zero block); a weight is twice its E2M1 value, an int8 in [-12, 12]; the
// 32-term integer dot of a block is exact and is scaled in fp32 by 2^(scale byte - 127) * s / 2. Mode "exact"
// (cpumoe_set_int8(0)) dequantises the weights to fp32 and accumulates x * w in fp32 instead. In both modes a
// scale byte of 0 contributes 0 (2^-127 is flushed), as in the reference CPU library (moe_cpu.cpp:186,270).
//
// Deviation from the reference, on purpose: stage 2 covers every column of h. The reference walks h in blocks
// of 256 columns (moe_cpu.cpp:444-450), so for I = 1664 (DeepSeek-V4's moe_inter_dim) its last 128 columns of
// each expert are never computed and stage 3 reads stale memory there.
//
// Design of this library:
//  * int8 kernel. The reference pays for unsigned-times-signed VNNI (vpdpbusd) by storing q + 128 and
//    subtracting 128 * sum(w) with two more dot products per row. Here the activation is stored as |q| (u8)
//    and its sign is folded into the weight: E2M1 is sign-magnitude, so negating the weight is flipping bit 3
//    of its nibble, one XOR of the packed bytes with a precomputed mask before the table lookup (vpermb, which
//    reads only the low 6 index bits, so no masking of the nibbles is needed either). Per 128 k and row:
//    1 shift, 2 XOR, 2 vpermb, 2 vpdpbusd, then a lane permute of the per-block scales and one FMA.
//  * 4 rows per pass share each activation load; the 16 block scales of a 512-k group are built once per row.
//  * Threads: a persistent pool, one worker pinned per listed CPU (numbered node by node), that spins between
//    calls for a bounded time and then sleeps on a condition variable; the caller waits. Rows of a matrix are
//    split by NUMA node (each node reads the rows it first-touched) and handed out within the node through one
//    atomic counter per node, in chunks of whole 4-row groups.
//  * Row order of every reduction is fixed (a row's dot product is computed by one thread, experts are summed
//    in selection order), so results do not depend on the thread count or on scheduling.
#include <immintrin.h>
#include <pthread.h>
#include <sched.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <sys/mman.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <mutex>
#include <thread>
#include <vector>

#include "dsv41_cpu.h"

namespace {

// ------------------------------------------------------------------------------------------- tables
// twice the E2M1 value of code (i & 15); vpermb indexes with the low 6 bits of each byte
alignas(64) const int8_t kLutW2[64] = {
    0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12, 0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12,
    0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12, 0, 1, 2, 3, 4, 6, 8, 12, 0, -1, -2, -3, -4, -6, -8, -12};
// the E2M1 value of code i (quant.py:24)
alignas(64) const float kLutF[16] = {0.f, .5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f, -0.f, -.5f, -1.f, -1.5f, -2.f, -3.f, -4.f, -6.f};
// 128-k chunk c of a 512-k group: int32 lane j of the chunk's dot products covers k [8j, 8j + 8), i.e. block 4c + j/4
alignas(64) const int32_t kLaneBlock[4][16] = {
    {0, 0, 0, 0, 1, 1, 1, 1, 2, 2, 2, 2, 3, 3, 3, 3},
    {4, 4, 4, 4, 5, 5, 5, 5, 6, 6, 6, 6, 7, 7, 7, 7},
    {8, 8, 8, 8, 9, 9, 9, 9, 10, 10, 10, 10, 11, 11, 11, 11},
    {12, 12, 12, 12, 13, 13, 13, 13, 14, 14, 14, 14, 15, 15, 15, 15}};

inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
inline float bf16_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }
inline uint16_t f32_bf16(float f) {   // round to nearest even (finite inputs)
    const uint32_t u = f32_bits(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
inline float bf16_round(float f) { return bf16_f32(f32_bf16(f)); }
inline float e8m0_f32(uint8_t b) { return bits_f32((uint32_t)b << 23); }   // byte 0 -> 0

// 2^k as fp32 for -126 <= k <= 127
inline float pow2f(int k) { return bits_f32((uint32_t)(k + 127) << 23); }

// ceil(log2(a)) for a finite a > 0, exactly (quant.py:34-37): the exponent, plus one unless a is a power of two
inline int ceil_log2(float a) {
    const uint32_t u = f32_bits(a);
    const int ef = (int)(u >> 23);
    if (ef == 0) {   // subnormal
        int e;
        const float m = frexpf(a, &e);
        return m == 0.5f ? e - 1 : e;
    }
    return ef - 127 + ((u & 0x7FFFFFu) != 0u);
}

// |v| rounded to E4M3 (3 mantissa bits, RNE, subnormal step 2^-9, saturating at 448), sign restored
inline float round_e4m3(float v) {
    const float a = fabsf(v);
    if (a == 0.f) return v;
    const int e = std::max((int)(f32_bits(a) >> 23) - 127, -6);   // floor(log2 a), at least the smallest normal exponent
    const float r = std::min(rintf(a * pow2f(3 - e)) * pow2f(e - 3), 448.f);   // scaling by powers of two is exact
    return v < 0.f ? -r : r;
}

// ------------------------------------------------------------------------------------------- thread pool
constexpr int kMaxNodes = 16;

class Pool {
public:
    int n = 0, per_node = 1, nodes = 1;
    std::vector<int> cpus;

    ~Pool() { stop(); }

    int start(const int* list, int count, int cores_per_node) {
        stop();
        n = count;
        per_node = std::max(1, std::min(cores_per_node, count));
        per_node = std::max(per_node, (count + kMaxNodes - 1) / kMaxNodes);   // at most kMaxNodes work queues
        nodes = (n + per_node - 1) / per_node;
        cpus.assign(list, list + count);
        const char* sp = getenv("DSV41_CPU_SPIN_US");
        spin_us_ = sp ? atoi(sp) : 2000;
        quit_.store(false);
        pinned_.store(0);
        first_run_ = true;
        const unsigned g0 = gen_.load();   // workers wait for the next generation, not a stale one
        for (int t = 1; t < n; ++t) th_.emplace_back([this, t, g0] { loop(t, g0); });
        // every worker has pinned itself (or failed to) once this empty job returns
        run([](void*, int) {}, nullptr);
        return n;
    }

    void stop() {
        if (n == 0) return;
        quit_.store(true);
        wake();
        for (auto& t : th_) t.join();
        th_.clear();
        n = 0;
    }

    // fn(ctx, t) on every worker t = 0..n-1 and returns when all have finished. The calling thread is worker 0:
    // it is pinned to cpus[0] for the call and gets its own affinity mask back afterwards.
    void run(void (*fn)(void*, int), void* ctx) {
        fn_ = fn;
        ctx_ = ctx;
        done_.store(0, std::memory_order_relaxed);
        wake();
        cpu_set_t saved, one;
        const bool have = pthread_getaffinity_np(pthread_self(), sizeof(saved), &saved) == 0;
        CPU_ZERO(&one);
        CPU_SET(cpus[0], &one);
        const bool pin = have && pthread_setaffinity_np(pthread_self(), sizeof(one), &one) == 0;
        if (first_run_) {
            first_run_ = false;
            if (pin) pinned_.fetch_add(1);
        }
        fn(ctx, 0);
        while (done_.load(std::memory_order_acquire) < n - 1) _mm_pause();
        if (pin) pthread_setaffinity_np(pthread_self(), sizeof(saved), &saved);
    }

    // all n workers of the running job meet here
    void barrier() {
        const unsigned g = bar_gen_.load(std::memory_order_acquire);
        if (bar_count_.fetch_add(1, std::memory_order_acq_rel) + 1 == n) {
            bar_count_.store(0, std::memory_order_relaxed);
            bar_gen_.fetch_add(1, std::memory_order_release);
        } else {
            while (bar_gen_.load(std::memory_order_acquire) == g) _mm_pause();
        }
    }

    int node_of(int t) const { return t / per_node; }
    int rank_in_node(int t) const { return t % per_node; }
    int threads_of_node(int k) const { return std::min(per_node, n - k * per_node); }
    int pinned() const { return pinned_.load(); }

private:
    void wake() {
        gen_.fetch_add(1, std::memory_order_seq_cst);
        if (sleepers_.load(std::memory_order_seq_cst) > 0) {
            { std::lock_guard<std::mutex> lk(mu_); }
            cv_.notify_all();
        }
    }

    void loop(int t, unsigned seen) {
        cpu_set_t set;
        CPU_ZERO(&set);
        CPU_SET(cpus[t], &set);
        if (pthread_setaffinity_np(pthread_self(), sizeof(set), &set) == 0) pinned_.fetch_add(1);
        for (;;) {
            unsigned g;
            auto t0 = std::chrono::steady_clock::now();
            int it = 0;
            while ((g = gen_.load(std::memory_order_acquire)) == seen) {
                _mm_pause();
                if ((++it & 255) == 0 &&
                    std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0).count() > spin_us_) {
                    sleepers_.fetch_add(1, std::memory_order_seq_cst);
                    {
                        std::unique_lock<std::mutex> lk(mu_);
                        cv_.wait(lk, [&] { return gen_.load(std::memory_order_seq_cst) != seen; });
                    }
                    sleepers_.fetch_sub(1, std::memory_order_seq_cst);
                }
            }
            seen = g;
            if (quit_.load()) return;
            fn_(ctx_, t);
            done_.fetch_add(1, std::memory_order_release);
        }
    }

    std::vector<std::thread> th_;
    void (*fn_)(void*, int) = nullptr;
    void* ctx_ = nullptr;
    int spin_us_ = 2000;
    bool first_run_ = true;
    std::atomic<bool> quit_{false};
    std::atomic<int> pinned_{0};
    alignas(64) std::atomic<unsigned> gen_{0};
    alignas(64) std::atomic<int> done_{0};
    alignas(64) std::atomic<int> sleepers_{0};
    alignas(64) std::atomic<int> bar_count_{0};
    alignas(64) std::atomic<unsigned> bar_gen_{0};
    std::mutex mu_;
    std::condition_variable cv_;
};

Pool g_pool;
std::mutex g_call;               // one entry point at a time: the pool and the workspace are shared
int g_mode = 2;                  // 0: exact fp32, otherwise int8
// rows per pass of the dot kernels: 8 streams per thread keep more DRAM requests in flight than 4 (measured on
// the EPYC host: 568-570 vs 620 us per configs[1] layer)
#ifndef DSV41_ROWS
#define DSV41_ROWS 8
#endif
constexpr int kRows = DSV41_ROWS;
static_assert(kRows == 1 || kRows == 2 || kRows == 4 || kRows == 8 || kRows == 16, "rows per pass: a power of two");
int g_ch1 = 192, g_ch3 = 128;    // largest row chunk handed out at once (stage 1 / stage 3)
int g_pf = 8192;                 // software prefetch distance along a weight row, bytes (0: none)

void ensure_pool() {
    if (g_pool.n > 0) return;
    const int hw = (int)std::max(1u, std::thread::hardware_concurrency());
    std::vector<int> list;
    cpu_set_t set;
    if (sched_getaffinity(0, sizeof(set), &set) == 0)
        for (int c = 0; c < CPU_SETSIZE && (int)list.size() < hw; ++c)
            if (CPU_ISSET(c, &set)) list.push_back(c);
    if (list.empty())
        for (int c = 0; c < hw; ++c) list.push_back(c);
    g_pool.start(list.data(), (int)list.size(), (int)list.size());
}

// ------------------------------------------------------------------------------------------- NUMA helpers
constexpr int kMpolDefault = 0, kMpolBind = 2;
void bind_self_node(int node) {
    if (g_pool.nodes <= 1) return;
    unsigned long mask = 1UL << node;
    syscall(SYS_set_mempolicy, kMpolBind, &mask, 64);
}
void unbind_self() {
    if (g_pool.nodes <= 1) return;
    syscall(SYS_set_mempolicy, kMpolDefault, nullptr, 0);
}
// rows [lo, hi) of an N-row matrix that node k reads
inline void node_rows(int N, int k, int nodes, int& lo, int& hi) {
    lo = (int)((long long)N * k / nodes);
    hi = (int)((long long)N * (k + 1) / nodes);
}

// ------------------------------------------------------------------------------------------- workspace
// An activation vector of K elements in the int8 form the kernels read: byte i of ae / ao holds |q| of element
// 2i / 2i + 1 and byte i of se / so holds 0x08 when that q is negative; sc[b] = s_b / 2 for block b (zero-padded
// to a multiple of 16 blocks). The exact mode reads fe / fo, the fp32 values of the even / odd elements.
struct Act {
    uint8_t* ae; uint8_t* ao; uint8_t* se; uint8_t* so;
    float* sc;
    float* fe; float* fo;
};

struct Buf {
    void* p = nullptr;
    size_t cap = 0;
    void* get(size_t bytes) {
        if (bytes > cap) {
            free(p);
            cap = (bytes + 4095) & ~(size_t)4095;
            p = aligned_alloc(64, cap);
            if (!p) cap = 0;
        }
        return p;
    }
};
Buf g_xbuf, g_hbuf;

// carve one Act for K elements (K % 32 == 0) from p; returns the bytes used (multiple of 64)
size_t act_bytes(int K) {
    const size_t half = ((size_t)K / 2 + 63) & ~(size_t)63;
    const size_t blocks = (((size_t)K / 32 + 15) & ~(size_t)15) * 4;
    const size_t fl = ((size_t)K / 2 * 4 + 63) & ~(size_t)63;
    return 4 * half + blocks + 2 * fl;
}
Act act_at(uint8_t* p, int K) {
    const size_t half = ((size_t)K / 2 + 63) & ~(size_t)63;
    const size_t blocks = (((size_t)K / 32 + 15) & ~(size_t)15) * 4;
    const size_t fl = ((size_t)K / 2 * 4 + 63) & ~(size_t)63;
    Act a;
    a.ae = p; a.ao = p + half; a.se = p + 2 * half; a.so = p + 3 * half;
    a.sc = (float*)(p + 4 * half);
    a.fe = (float*)(p + 4 * half + blocks);
    a.fo = (float*)(p + 4 * half + blocks + fl);
    return a;
}

// the scale padding past the last block is read (and multiplied by a zero weight scale): keep it finite
void act_clear_pad(const Act& a, int K) {
    const int nb = K / 32, padded = (nb + 15) & ~15;
    for (int b = nb; b < padded; ++b) a.sc[b] = 0.f;
}

// block b (32 values v) of an activation into its int8 (mode != 0) or fp32 form (quant_x_u8, moe_cpu.cpp:218-228)
alignas(64) const int32_t kEven[16] = {0, 2, 4, 6, 8, 10, 12, 14, 16, 18, 20, 22, 24, 26, 28, 30};
alignas(64) const int32_t kOdd[16] = {1, 3, 5, 7, 9, 11, 13, 15, 17, 19, 21, 23, 25, 27, 29, 31};

inline void act_block(const float* v, int b, const Act& a, int mode) {
    const __m512 v0 = _mm512_loadu_ps(v), v1 = _mm512_loadu_ps(v + 16);
    const __m512i ie = _mm512_load_si512(kEven), io = _mm512_load_si512(kOdd);
    if (mode == 0) {
        _mm512_storeu_ps(a.fe + 16 * b, _mm512_permutex2var_ps(v0, ie, v1));
        _mm512_storeu_ps(a.fo + 16 * b, _mm512_permutex2var_ps(v0, io, v1));
        return;
    }
    const float amax = _mm512_reduce_max_ps(_mm512_max_ps(_mm512_abs_ps(v0), _mm512_abs_ps(v1)));
    const float s = amax > 0.f ? amax / 127.f : 1.f;
    const __m512 inv = _mm512_set1_ps(1.f / s);
    const __m512i lo = _mm512_set1_epi32(-127), hi = _mm512_set1_epi32(127);
    // v * (1 / s) rounded to nearest even (the MXCSR default, as rintf), then clamped
    const __m512i q0 = _mm512_min_epi32(_mm512_max_epi32(_mm512_cvtps_epi32(_mm512_mul_ps(v0, inv)), lo), hi);
    const __m512i q1 = _mm512_min_epi32(_mm512_max_epi32(_mm512_cvtps_epi32(_mm512_mul_ps(v1, inv)), lo), hi);
    const __m512i qe = _mm512_permutex2var_epi32(q0, ie, q1), qo = _mm512_permutex2var_epi32(q0, io, q1);
    const __m128i eight = _mm_set1_epi8(0x08);
    _mm_storeu_si128((__m128i*)(a.ae + 16 * b), _mm512_cvtepi32_epi8(_mm512_abs_epi32(qe)));
    _mm_storeu_si128((__m128i*)(a.ao + 16 * b), _mm512_cvtepi32_epi8(_mm512_abs_epi32(qo)));
    _mm_storeu_si128((__m128i*)(a.se + 16 * b), _mm_maskz_mov_epi8(_mm512_cmplt_epi32_mask(qe, _mm512_setzero_si512()), eight));
    _mm_storeu_si128((__m128i*)(a.so + 16 * b), _mm_maskz_mov_epi8(_mm512_cmplt_epi32_mask(qo, _mm512_setzero_si512()), eight));
    a.sc[b] = s * 0.5f;   // the weights enter as twice their value
}

// 32 bf16 values at x into fp32
inline void bf16x32(const uint16_t* x, float* v) {
    const __m512i w = _mm512_loadu_si512(x);
    _mm512_storeu_ps(v, _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(_mm512_castsi512_si256(w)), 16)));
    _mm512_storeu_ps(v + 16, _mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu16_epi32(_mm512_extracti64x4_epi64(w, 1)), 16)));
}

// ------------------------------------------------------------------------------------------- dot kernels
// R rows (packed E2M1 [K/2], E8M0 [K/32]) against one int8 activation; K % 128 == 0
template <int R>
inline void dot_i8(const uint8_t* const* w, const uint8_t* const* s, const Act& a, int K, float* res) {
    const __m512i lut = _mm512_load_si512(kLutW2);
    __m512 acc[R];
    for (int r = 0; r < R; ++r) acc[r] = _mm512_setzero_ps();
    const int nblk = K >> 5;
    const int pf = g_pf;
    for (int kb = 0; kb < nblk; kb += 16) {
        const int nb = std::min(16, nblk - kb);
        const __mmask16 m = (__mmask16)((1u << nb) - 1u);
        const __m512 xs = _mm512_load_ps(a.sc + kb);
        __m512 sv[R];
        for (int r = 0; r < R; ++r)
            sv[r] = _mm512_mul_ps(_mm512_castsi512_ps(_mm512_slli_epi32(_mm512_cvtepu8_epi32(_mm_maskz_loadu_epi8(m, s[r] + kb)), 23)), xs);
        for (int c = 0; c < (nb >> 2); ++c) {
            const size_t o = (size_t)(kb + 4 * c) * 16;   // byte offset of this 128-k chunk
            const __m512i xe = _mm512_load_si512(a.ae + o), xo = _mm512_load_si512(a.ao + o);
            const __m512i se = _mm512_load_si512(a.se + o), so = _mm512_load_si512(a.so + o);
            const __m512i li = _mm512_load_si512(kLaneBlock[c]);
            for (int r = 0; r < R; ++r) {
                if (pf) _mm_prefetch((const char*)(w[r] + o + pf), _MM_HINT_T0);
                const __m512i p = _mm512_loadu_si512(w[r] + o);
                const __m512i wl = _mm512_permutexvar_epi8(_mm512_xor_si512(p, se), lut);
                const __m512i wh = _mm512_permutexvar_epi8(_mm512_xor_si512(_mm512_srli_epi16(p, 4), so), lut);
                const __m512i d = _mm512_dpbusd_epi32(_mm512_dpbusd_epi32(_mm512_setzero_si512(), xe, wl), xo, wh);
                acc[r] = _mm512_fmadd_ps(_mm512_cvtepi32_ps(d), _mm512_permutexvar_ps(li, sv[r]), acc[r]);
            }
        }
    }
    for (int r = 0; r < R; ++r) res[r] = _mm512_reduce_add_ps(acc[r]);
}

// R rows against one fp32 activation (exact mode); K % 32 == 0
template <int R>
inline void dot_f32(const uint8_t* const* w, const uint8_t* const* s, const Act& a, int K, float* res) {
    const __m512 lut = _mm512_load_ps(kLutF);
    const __m512i m4 = _mm512_set1_epi32(15);
    __m512 acc[R];
    for (int r = 0; r < R; ++r) acc[r] = _mm512_setzero_ps();
    const int pf = g_pf;
    for (int b = 0; b < (K >> 5); ++b) {
        const __m512 xe = _mm512_loadu_ps(a.fe + 16 * b), xo = _mm512_loadu_ps(a.fo + 16 * b);
        for (int r = 0; r < R; ++r) {
            if (pf) _mm_prefetch((const char*)(w[r] + 16 * b + pf), _MM_HINT_T0);
            const __m512i p = _mm512_cvtepu8_epi32(_mm_loadu_si128((const __m128i*)(w[r] + 16 * b)));
            const __m512 we = _mm512_permutexvar_ps(_mm512_and_si512(p, m4), lut);
            const __m512 wo = _mm512_permutexvar_ps(_mm512_srli_epi32(p, 4), lut);
            const __m512 t = _mm512_fmadd_ps(wo, xo, _mm512_mul_ps(we, xe));   // products are exact
            acc[r] = _mm512_fmadd_ps(t, _mm512_set1_ps(e8m0_f32(s[r][b])), acc[r]);
        }
    }
    for (int r = 0; r < R; ++r) res[r] = _mm512_reduce_add_ps(acc[r]);
}

// rows [a, b) of a row-major matrix (row_bytes = K / 2, srow = K / 32) into out[0 .. b - a)
void dot_rows(const uint8_t* W, const uint8_t* S, int a, int b, const Act& x, int K, int mode, float* out) {
    const size_t rb = (size_t)K / 2, rs = (size_t)K / 32;
    int n = a;
    constexpr int R = kRows;
    for (; n + R <= b; n += R) {
        const uint8_t* w[R];
        const uint8_t* s[R];
        for (int r = 0; r < R; ++r) { w[r] = W + (n + r) * rb; s[r] = S + (n + r) * rs; }
        if (mode) dot_i8<R>(w, s, x, K, out + (n - a));
        else dot_f32<R>(w, s, x, K, out + (n - a));
    }
    for (; n < b; ++n) {
        const uint8_t* w[1] = {W + n * rb};
        const uint8_t* s[1] = {S + n * rs};
        if (mode) dot_i8<1>(w, s, x, K, out + (n - a));
        else dot_f32<1>(w, s, x, K, out + (n - a));
    }
}

// ------------------------------------------------------------------------------------------- layer forward
struct Layer {
    const uint8_t* const* w13; const uint8_t* const* s13; const uint8_t* const* w2; const uint8_t* const* s2;
    int E;
    const uint16_t* x;
    const float* wts;
    float* out;
    int K, inter, dim;
    float limit;
    float* gu;
    uint16_t* h;
    int mode;
    Act xa;
    uint8_t* hbase;        // E activations of `inter` elements, act_bytes(inter) apart
    size_t hstride;
    alignas(64) std::atomic<int> ctr1[kMaxNodes * 16];   // per-node work counters, one cache line each
    alignas(64) std::atomic<int> ctr3[kMaxNodes * 16];
};

Act h_act(const Layer& L, int e) { return act_at(L.hbase + (size_t)e * L.hstride, L.inter); }

// largest chunk of rows (a multiple of kRows) that still gives every thread of a node about 8 work items
int chunk_rows(long long rows_total, int threads, int cap, int floor_rows) {
    long long c = rows_total / ((long long)threads * 8);
    c &= ~(long long)(kRows - 1);
    c = std::max<long long>(c, floor_rows);
    c = std::min<long long>(c, std::max(kRows, cap & ~(kRows - 1)));
    return (int)c;
}

void layer_job(void* p, int t) {
    Layer& L = *(Layer*)p;
    Pool& P = g_pool;
    const int node = P.node_of(t), tn = P.threads_of_node(node);
    const int K = L.K, I = L.inter, N13 = 2 * I, H = L.dim;

    // stage 0: x into its int8 / fp32 form, blocks split over all threads
    {
        const int nb = K / 32;
        const int per = (nb + P.n - 1) / P.n;
        float v[32];
        for (int b = t * per; b < std::min(nb, (t + 1) * per); ++b) {
            bf16x32(L.x + 32 * b, v);
            act_block(v, b, L.xa, L.mode);
        }
    }
    P.barrier();

    // stage 1: gu[e][n] = x . W13[e][n], this node's rows of every selected expert
    {
        int n0, n1;
        node_rows(N13, node, P.nodes, n0, n1);
        const int CH = chunk_rows((long long)(n1 - n0) * L.E, tn, g_ch1, 32);
        const int nch = (n1 - n0 + CH - 1) / CH, total = L.E * nch;
        for (;;) {
            const int c = L.ctr1[node * 16].fetch_add(1, std::memory_order_relaxed);
            if (c >= total) break;
            const int e = c / nch, a = n0 + (c % nch) * CH, b = std::min(a + CH, n1);
            dot_rows(L.w13[e], L.s13[e], a, b, L.xa, K, L.mode, L.gu + (size_t)e * N13 + a);
        }
    }
    P.barrier();

    // stage 2: h[e] = fq8(bf16(wt * silu(g) * u)) per 32 columns (swiglu_quant_cols, moe_cpu.cpp:357-377),
    // every block of every expert (no 256-column tail loss); then h[e] into the stage-3 activation form
    {
        const int nbl = I / 32, total = L.E * nbl;
        const int per = (total + P.n - 1) / P.n;
        float v[32];
        for (int i = t * per; i < std::min(total, (t + 1) * per); ++i) {
            const int e = i / nbl, b = i % nbl;
            const float* g = L.gu + (size_t)e * N13 + 32 * b;
            const float* u = g + I;
            const float wt = L.wts[e];
            float amax = 1e-4f;   // quant.py's amax floor
            for (int j = 0; j < 32; ++j) {
                float gj = g[j], uj = u[j];
                if (L.limit > 0.f) {
                    uj = std::min(std::max(uj, -L.limit), L.limit);
                    gj = std::min(gj, L.limit);
                }
                const float r = bf16_round(wt * (gj / (1.f + expf(-gj))) * uj);
                v[j] = r;
                amax = std::max(amax, fabsf(r));
            }
            const float sc = pow2f(ceil_log2(amax / 448.f));
            uint16_t* hb = L.h + (size_t)e * I + 32 * b;
            for (int j = 0; j < 32; ++j) {
                const float q = std::min(std::max(v[j] / sc, -448.f), 448.f);
                hb[j] = f32_bf16(round_e4m3(q) * sc);
                v[j] = bf16_f32(hb[j]);
            }
            act_block(v, b, h_act(L, e), L.mode);
        }
    }
    P.barrier();

    // stage 3: out[n] = sum_e h[e] . W2[e][n], this node's output rows in chunks; experts outer inside a chunk
    {
        int n0, n1;
        node_rows(H, node, P.nodes, n0, n1);
        const int CH = chunk_rows(n1 - n0, tn, std::min(g_ch3, 256), 16);
        const int nch = (n1 - n0 + CH - 1) / CH;
        alignas(64) float acc[256], part[256];
        for (;;) {
            const int c = L.ctr3[node * 16].fetch_add(1, std::memory_order_relaxed);
            if (c >= nch) break;
            const int a = n0 + c * CH, b = std::min(a + CH, n1);
            for (int i = 0; i < b - a; ++i) acc[i] = 0.f;
            for (int e = 0; e < L.E; ++e) {
                dot_rows(L.w2[e], L.s2[e], a, b, h_act(L, e), I, L.mode, part);
                for (int i = 0; i < b - a; ++i) acc[i] += part[i];
            }
            memcpy(L.out + a, acc, sizeof(float) * (size_t)(b - a));
        }
    }
}

bool mode_shape_ok(int K, int mode) { return K > 0 && (mode ? K % 128 == 0 : K % 32 == 0); }

// ------------------------------------------------------------------------------------------- single GEMV
struct Gemv {
    const uint8_t* w; const uint8_t* s;
    int N, K;
    const uint16_t* x;
    float* out;
    int mode;
    Act xa;
    int CH;
    alignas(64) std::atomic<int> ctr{0};
};

void gemv_job(void* p, int t) {
    Gemv& G = *(Gemv*)p;
    Pool& P = g_pool;
    const int nb = G.K / 32, per = (nb + P.n - 1) / P.n;
    float v[32];
    for (int b = t * per; b < std::min(nb, (t + 1) * per); ++b) {
        bf16x32(G.x + 32 * b, v);
        act_block(v, b, G.xa, G.mode);
    }
    P.barrier();
    const int nch = (G.N + G.CH - 1) / G.CH;
    for (;;) {
        const int c = G.ctr.fetch_add(1, std::memory_order_relaxed);
        if (c >= nch) break;
        const int a = c * G.CH, b = std::min(a + G.CH, G.N);
        dot_rows(G.w, G.s, a, b, G.xa, G.K, G.mode, G.out + a);
    }
}

// ------------------------------------------------------------------------------------------- copies
struct Copy {
    // load_rows
    uint8_t* dst; const uint8_t* src; int N; int row_bytes;
    // load_expert / load_layer
    uint8_t *w13, *s13, *w2, *s2;
    int e, E, inter, dim;
    const uint8_t *sw1, *sw3, *ss1, *ss3, *sw2, *ss2;                          // one expert
    const uint8_t* const *lw1, *const *lw3, *const *ls1, *const *ls3, *const *lw2, *const *ls2;   // a layer
};

// rows [a, b) of this thread's share: node k's rows split evenly among its threads
void thread_rows(int N, int t, int& a, int& b) {
    const Pool& P = g_pool;
    const int node = P.node_of(t), tin = P.rank_in_node(t), tn = P.threads_of_node(node);
    int n0, n1;
    node_rows(N, node, P.nodes, n0, n1);
    const int per = (n1 - n0 + tn - 1) / tn;
    a = std::min(n1, n0 + tin * per);
    b = std::min(n1, a + per);
}

// row n of the [w1; w3] stack of one expert: w1 rows first
inline void copy_w13_rows(const Copy& C, int e, const uint8_t* w1, const uint8_t* w3, const uint8_t* s1, const uint8_t* s3, int a, int b) {
    const size_t rb = (size_t)C.dim / 2, rs = (size_t)C.dim / 32, N13 = 2 * (size_t)C.inter;
    for (int n = a; n < b;) {
        const bool up = n >= C.inter;
        const int end = up ? b : std::min(b, C.inter);
        const size_t r0 = up ? n - C.inter : n;
        memcpy(C.w13 + ((size_t)e * N13 + n) * rb, (up ? w3 : w1) + r0 * rb, (size_t)(end - n) * rb);
        memcpy(C.s13 + ((size_t)e * N13 + n) * rs, (up ? s3 : s1) + r0 * rs, (size_t)(end - n) * rs);
        n = end;
    }
}

inline void copy_w2_rows(const Copy& C, int e, const uint8_t* w2, const uint8_t* s2, int a, int b) {
    const size_t rb = (size_t)C.inter / 2, rs = (size_t)C.inter / 32;
    if (a >= b) return;
    memcpy(C.w2 + ((size_t)e * C.dim + a) * rb, w2 + (size_t)a * rb, (size_t)(b - a) * rb);
    memcpy(C.s2 + ((size_t)e * C.dim + a) * rs, s2 + (size_t)a * rs, (size_t)(b - a) * rs);
}

void load_rows_job(void* p, int t) {
    const Copy& C = *(const Copy*)p;
    int a, b;
    thread_rows(C.N, t, a, b);
    bind_self_node(g_pool.node_of(t));
    if (a < b) memcpy(C.dst + (size_t)a * C.row_bytes, C.src + (size_t)a * C.row_bytes, (size_t)(b - a) * C.row_bytes);
    unbind_self();
}

void load_expert_job(void* p, int t) {
    const Copy& C = *(const Copy*)p;
    bind_self_node(g_pool.node_of(t));
    int a, b;
    thread_rows(2 * C.inter, t, a, b);
    copy_w13_rows(C, C.e, C.sw1, C.sw3, C.ss1, C.ss3, a, b);
    thread_rows(C.dim, t, a, b);
    copy_w2_rows(C, C.e, C.sw2, C.ss2, a, b);
    unbind_self();
}

// a whole layer: each node copies its own row halves, its threads taking the experts in turn
void load_layer_job(void* p, int t) {
    const Copy& C = *(const Copy*)p;
    const Pool& P = g_pool;
    const int node = P.node_of(t), tin = P.rank_in_node(t), tn = P.threads_of_node(node);
    bind_self_node(node);
    int a13, z13, a2, z2;
    node_rows(2 * C.inter, node, P.nodes, a13, z13);
    node_rows(C.dim, node, P.nodes, a2, z2);
    for (int e = tin; e < C.E; e += tn) {
        copy_w13_rows(C, e, C.lw1[e], C.lw3[e], C.ls1[e], C.ls3[e], a13, z13);
        copy_w2_rows(C, e, C.lw2[e], C.ls2[e], a2, z2);
    }
    unbind_self();
}

struct Bw {
    const uint8_t* p; size_t bytes; int node_sel;
    alignas(64) long long sink[256];
};

void bw_job(void* q, int t) {
    Bw& B = *(Bw*)q;
    const Pool& P = g_pool;
    const int node = P.node_of(t), tin = P.rank_in_node(t), tn = P.threads_of_node(node);
    if (B.node_sel >= 0 && node != B.node_sel) return;
    const size_t b0 = B.bytes * node / P.nodes, b1 = B.bytes * (node + 1) / P.nodes;
    const size_t per = ((b1 - b0) / tn) & ~(size_t)63;
    const uint8_t* a = B.p + b0 + tin * per;
    __m512i s0 = _mm512_setzero_si512(), s1 = s0, s2 = s0, s3 = s0;
    size_t i = 0;
    // the same software prefetch distance as the expert kernels' weight streams (g_pf bytes ahead), so the probe
    // measures what a core's stream can draw, not the hardware prefetcher's reach alone
    const size_t pf = (size_t)g_pf;
    for (; i + 256 <= per; i += 256) {
        if (pf && i + pf + 256 <= per) {
            _mm_prefetch((const char*)(a + i + pf), _MM_HINT_T0);
            _mm_prefetch((const char*)(a + i + pf + 64), _MM_HINT_T0);
            _mm_prefetch((const char*)(a + i + pf + 128), _MM_HINT_T0);
            _mm_prefetch((const char*)(a + i + pf + 192), _MM_HINT_T0);
        }
        s0 = _mm512_add_epi64(s0, _mm512_loadu_si512(a + i));
        s1 = _mm512_add_epi64(s1, _mm512_loadu_si512(a + i + 64));
        s2 = _mm512_add_epi64(s2, _mm512_loadu_si512(a + i + 128));
        s3 = _mm512_add_epi64(s3, _mm512_loadu_si512(a + i + 192));
    }
    for (; i + 64 <= per; i += 64) s0 = _mm512_add_epi64(s0, _mm512_loadu_si512(a + i));
    B.sink[t & 255] = _mm512_reduce_add_epi64(_mm512_add_epi64(_mm512_add_epi64(s0, s1), _mm512_add_epi64(s2, s3)));
}

}  // namespace

// =========================================================================================== C ABI
extern "C" {

void cpumoe_init(int threads, int cores_per_node) {
    std::lock_guard<std::mutex> lk(g_call);
    threads = std::max(1, std::min(threads, 256));
    std::vector<int> list(threads);
    for (int t = 0; t < threads; ++t) list[t] = t;
    g_pool.start(list.data(), threads, cores_per_node > 0 ? cores_per_node : threads);
}

int cpumoe_init_list(const int* cpus, int n, int cores_per_node) {
    std::lock_guard<std::mutex> lk(g_call);
    if (!cpus || n < 1 || n > 256) return 0;
    return g_pool.start(cpus, n, cores_per_node > 0 ? cores_per_node : n);
}

int cpumoe_threads_pinned(void) { return g_pool.pinned(); }

void* cpumoe_alloc(size_t bytes) {
    void* p = mmap(nullptr, bytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (p == MAP_FAILED) return nullptr;
    if (!getenv("DSV41_NO_THP")) madvise(p, bytes, MADV_HUGEPAGE);
    return p;
}

int cpumoe_free(void* p, size_t bytes) { return p ? munmap(p, bytes) : 0; }

int cpumoe_bind_rows(uint8_t* base, int E, int N, int row_bytes) {
    std::lock_guard<std::mutex> lk(g_call);
    ensure_pool();
    if (g_pool.nodes <= 1) return 0;
    const uintptr_t page = (uintptr_t)sysconf(_SC_PAGESIZE);
    int bad = 0;
    for (int e = 0; e < E; ++e)
        for (int k = 0; k < g_pool.nodes; ++k) {
            int n0, n1;
            node_rows(N, k, g_pool.nodes, n0, n1);
            uintptr_t a = (uintptr_t)base + ((size_t)e * N + n0) * (size_t)row_bytes;
            uintptr_t b = (uintptr_t)base + ((size_t)e * N + n1) * (size_t)row_bytes;
            a = (a + page - 1) & ~(page - 1);
            b &= ~(page - 1);
            if (b <= a) continue;
            unsigned long mask = 1UL << k;
            if (syscall(SYS_mbind, (void*)a, (size_t)(b - a), kMpolBind, &mask, 64, 0) != 0) ++bad;
        }
    return bad;
}

double cpumoe_local_fraction(const uint8_t* base, int E, int N, int row_bytes) {
    std::lock_guard<std::mutex> lk(g_call);
    ensure_pool();
    const size_t huge = (size_t)2 << 20;
    long long ok = 0, tot = 0;
    for (int e = 0; e < E; ++e)
        for (int k = 0; k < g_pool.nodes; ++k) {
            int n0, n1;
            node_rows(N, k, g_pool.nodes, n0, n1);
            const uintptr_t a = (uintptr_t)base + ((size_t)e * N + n0) * (size_t)row_bytes;
            const uintptr_t b = (uintptr_t)base + ((size_t)e * N + n1) * (size_t)row_bytes;
            for (uintptr_t q = (a + huge - 1) & ~(uintptr_t)(huge - 1); q + huge <= b; q += huge) {
                void* pages[1] = {(void*)q};
                int status[1] = {-1};
                if (syscall(SYS_move_pages, 0, 1UL, pages, nullptr, status, 0) == 0 && status[0] >= 0) {
                    ++tot;
                    ok += status[0] == k;
                }
            }
        }
    return tot ? (double)ok / (double)tot : -1.0;
}

void cpumoe_load_rows(uint8_t* dst, const uint8_t* src, int N, int row_bytes) {
    std::lock_guard<std::mutex> lk(g_call);
    ensure_pool();
    Copy C{};
    C.dst = dst; C.src = src; C.N = N; C.row_bytes = row_bytes;
    g_pool.run(load_rows_job, &C);
}

void cpumoe_load_expert(uint8_t* w13, uint8_t* s13, uint8_t* w2, uint8_t* s2, int e, const uint8_t* src_w1, const uint8_t* src_w3,
                        const uint8_t* src_s1, const uint8_t* src_s3, const uint8_t* src_w2, const uint8_t* src_s2, int inter, int dim) {
    std::lock_guard<std::mutex> lk(g_call);
    ensure_pool();
    Copy C{};
    C.w13 = w13; C.s13 = s13; C.w2 = w2; C.s2 = s2; C.e = e; C.inter = inter; C.dim = dim;
    C.sw1 = src_w1; C.sw3 = src_w3; C.ss1 = src_s1; C.ss3 = src_s3; C.sw2 = src_w2; C.ss2 = src_s2;
    g_pool.run(load_expert_job, &C);
}

void cpumoe_load_layer(uint8_t* w13, uint8_t* s13, uint8_t* w2, uint8_t* s2, const uint8_t* const* sw1, const uint8_t* const* sw3,
                       const uint8_t* const* ss1, const uint8_t* const* ss3, const uint8_t* const* sw2, const uint8_t* const* ss2,
                       int E, int inter, int dim) {
    std::lock_guard<std::mutex> lk(g_call);
    ensure_pool();
    Copy C{};
    C.w13 = w13; C.s13 = s13; C.w2 = w2; C.s2 = s2; C.E = E; C.inter = inter; C.dim = dim;
    C.lw1 = sw1; C.lw3 = sw3; C.ls1 = ss1; C.ls3 = ss3; C.lw2 = sw2; C.ls2 = ss2;
    g_pool.run(load_layer_job, &C);
}

double cpumoe_bw_test(const uint8_t* p, size_t bytes, int iters, int node_sel) {
    std::lock_guard<std::mutex> lk(g_call);
    ensure_pool();
    if (((uintptr_t)p & 63) || iters < 1) return 0.0;
    Bw B{};
    B.p = p; B.bytes = bytes; B.node_sel = node_sel;
    double best = 0.0;
    for (int it = 0; it < iters; ++it) {
        const auto t0 = std::chrono::steady_clock::now();
        g_pool.run(bw_job, &B);
        const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        const double read = node_sel < 0 ? (double)bytes : (double)bytes / g_pool.nodes;
        best = std::max(best, read / dt / 1e9);
    }
    return best;
}

void cpumoe_set_chunks(int ch1, int ch3) {
    g_ch1 = ch1 > 0 ? ch1 : 64;
    g_ch3 = ch3 > 0 && ch3 <= 256 ? ch3 : 64;
}

void cpumoe_set_int8(int on) { g_mode = on; }

void cpumoe_set_prefetch(int bytes) { g_pf = std::max(0, bytes); }

int cpumoe_forward(const uint8_t* const* w13, const uint8_t* const* s13, const uint8_t* const* w2, const uint8_t* const* s2, int E,
                   const uint16_t* x, const float* wts, float* out, int K, int inter, int dim, float limit, float* gu, uint16_t* h) {
    if (E > 16) return -1;
    if (E < 0 || !x || !out || dim <= 0 || !mode_shape_ok(K, g_mode) || !mode_shape_ok(inter, g_mode) || (E > 0 && (!w13 || !s13 || !w2 || !s2 || !wts || !gu || !h)))
        return -2;
    if (E == 0) {
        memset(out, 0, sizeof(float) * (size_t)dim);
        return 0;
    }
    std::lock_guard<std::mutex> lk(g_call);
    ensure_pool();
    Layer* L = new Layer();
    L->w13 = w13; L->s13 = s13; L->w2 = w2; L->s2 = s2; L->E = E; L->x = x; L->wts = wts; L->out = out;
    L->K = K; L->inter = inter; L->dim = dim; L->limit = limit; L->gu = gu; L->h = h; L->mode = g_mode;
    uint8_t* xb = (uint8_t*)g_xbuf.get(act_bytes(K));
    L->hstride = act_bytes(inter);
    L->hbase = (uint8_t*)g_hbuf.get(L->hstride * (size_t)E);
    if (!xb || !L->hbase) {
        delete L;
        return -3;
    }
    L->xa = act_at(xb, K);
    act_clear_pad(L->xa, K);
    for (int e = 0; e < E; ++e) act_clear_pad(h_act(*L, e), inter);
    for (auto& c : L->ctr1) c.store(0, std::memory_order_relaxed);
    for (auto& c : L->ctr3) c.store(0, std::memory_order_relaxed);
    g_pool.run(layer_job, L);
    delete L;
    return 0;
}

int cpumoe_forward_ids(const uint8_t* w13, const uint8_t* s13, const uint8_t* w2, const uint8_t* s2, size_t b13, size_t bs13, size_t b2,
                       size_t bs2, const int* ids, int E, const uint16_t* x, const float* wts, float* out, int K, int inter, int dim,
                       float limit, float* gu, uint16_t* h) {
    if (E > 16) return -1;
    if (E < 0 || (E > 0 && !ids)) return -2;
    const uint8_t *p13[16], *ps13[16], *p2[16], *ps2[16];
    for (int j = 0; j < E; ++j) {
        if (ids[j] < 0) return -2;
        p13[j] = w13 + (size_t)ids[j] * b13;
        ps13[j] = s13 + (size_t)ids[j] * bs13;
        p2[j] = w2 + (size_t)ids[j] * b2;
        ps2[j] = s2 + (size_t)ids[j] * bs2;
    }
    return cpumoe_forward(p13, ps13, p2, ps2, E, x, wts, out, K, inter, dim, limit, gu, h);
}

int cpumoe_gemv(const uint8_t* w, const uint8_t* s, int N, int K, const uint16_t* x, float* out) {
    if (!w || !s || !x || !out || N <= 0 || !mode_shape_ok(K, g_mode)) return -2;
    std::lock_guard<std::mutex> lk(g_call);
    ensure_pool();
    Gemv* G = new Gemv();
    G->w = w; G->s = s; G->N = N; G->K = K; G->x = x; G->out = out; G->mode = g_mode;
    uint8_t* xb = (uint8_t*)g_xbuf.get(act_bytes(K));
    if (!xb) {
        delete G;
        return -3;
    }
    G->xa = act_at(xb, K);
    act_clear_pad(G->xa, K);
    G->CH = chunk_rows(N, g_pool.n, 64, 16);
    g_pool.run(gemv_job, G);
    delete G;
    return 0;
}

}  // extern "C"
