// Prefill expert GEMMs on gfx950 block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4), for many tokens per
// expert (model.MoE.__call__ beyond 16 tokens, model.py:539-551, 584-589; moe_kernels.grouped_fp4_gemm,
// moe_kernels.py:127-200).
//
// The (token, expert) pairs arrive bucketed by expert in groups of <= 256 pairs (moe_dispatch tables, gmax 256; the
// reference-shaped grouped-GEMM surface: <= 128). One workgroup computes a 256-row x 128-pair tile of one group over
// the full K (groups of more than 128 pairs: a 256-row x 256-pair tile, below):
//   MODE 0 (w13): rows = 128 gate rows c0 .. c0 + 127 and the matching 128 up rows I + c0 .., so the epilogue
//          turns the tile into h = fq8(bf16(w * silu(min(g, L)) * clamp(u, +-L))) for 128 columns (four FP8
//          groups) of every pair (fused.py:284-306) -- gate/up never reach HBM;
//   MODE 1 (w2):  rows = 256 consecutive output rows; the epilogue stores fp32 y2[pair][row].
//   MODE 2:       MODE 1 adding into y2 instead of storing, for the second FP8 term of off-grid activations
//          (dsv41_quant_fp8_split); the launch returns at once when that term is all zero (*run_if == 0).
// The weight operand is the raw E2M1 nibbles + E8M0 bytes as stored; the activation operand the E4M3 codes of the
// group's tokens, gathered by token id.
// Workgroup order is XCD-aware: the hardware hands workgroup i to XCD i % 8. XCD x takes the groups g = x, x + 8,
// x + 16, ... and walks their column blocks column-block-fastest, so the column blocks of one group run together on
// one XCD and read the group's activations from that XCD's L2 (instead of once per column block from HBM), while the
// groups of a popular expert (full groups, the costly items) are spread over all eight XCDs.
#include "common.h"

#define PG_THREADS 512
#define PG_T 128                // pairs per tile
#define PG_PF 3                 // minimum k-steps (K >= 384)

struct PrefillArgs {
    const uint8_t* xc; long long ldx;        // E4M3 codes [rows][ldx]: activations (MODE 0) or h (MODE 1)
    const uint8_t* xs; long long ldxs;       // E8M0 [rows][ldxs]
    uint32_t xc_bytes, xs_bytes;             // rows * ldx, rows * ldxs (< 2^32: 32-bit buffer offsets)
    const uint8_t* W; long long stride_we;   // packed E2M1 [E][N][K/2] (tiled or row-major)
    const uint8_t* S; long long stride_se;
    int N, K, E;                              // N = weight rows (MODE 0: 2 I), K = reduction length
    const int* grp_expert; const int* grp_start; int G;
    const int* row_of_pair;                  // input row of sorted pair p (MODE 1: NULL = row p); rows outside the
                                             // buffer read zeros (buffer descriptors bound every activation load)
    const float* wt_sorted;                  // MODE 0: routing weight of sorted pair p
    float limit;
    uint8_t* hc; long long ldhc; uint8_t* hs; long long ldhs;   // MODE 0 outputs
    float* y; long long ldy;                                     // MODE 1 output fp32 [pairs][ldy]
    int n_cb;                                 // column blocks (MODE 0: I / 128, MODE 1: N / 256)
    int g_pad;                                // G rounded up to a multiple of 8 (XCD remap)
    int n_pairs;                              // group ranges are clamped to [0, n_pairs)
    int cbw, n_it;                            // column blocks per workgroup, workgroups per group (ceil(n_cb / cbw))
    const int* run_if;                        // MODE 2, optional: the launch does nothing when *run_if == 0
    const int* grp_order;                     // optional: the order the items take the groups in (dsv41_group_order)
};

// The group an item's group index stands for: the index itself, or its place in grp_order (largest groups first, so no
// long item starts near the end of the launch). An order entry outside [0, G) maps to G, which no item computes.
__device__ __forceinline__ int item_group(const PrefillArgs& a, int g) {
    if (!a.grp_order || g >= a.G) return g;
    const int o = a.grp_order[g];
    return (o >= 0 && o < a.G) ? o : a.G;
}

// ------------------------------------------------------------------------------------------ direct-to-LDS variant
// A 256-row x 128-pair tile (MODE 0: 128 gate rows + the matching 128 up rows = 128 SwiGLU columns; MODE 1: 256
// output rows). Doubling the rows per tile halves how often each activation byte is re-read (once per column
// block), which is what bounds the kernel once many tokens share an expert.
// Every operand moves HBM/L2 -> LDS through the load unit itself (buffer_load ... lds, all through buffer descriptors):
// no staging registers, PV_NS k-steps (PV_NS x 33 KB) in flight per workgroup. Per k-step, with wave-uniform
// branches only: wave w loads weight slots 2 w, 2 w + 1 (1 KB each, 16 B per lane) and token block w (two 1 KB
// halves); the E8M0 bytes of the 16 weight slots (tiled: wave 0, 16 B per lane; row-major: waves 0-3, 4 slots each);
// waves 4-5 the E8M0 words of 64 pairs each.
// A wave waits for its own loads with vmcnt (they complete in order), then a barrier makes every wave's part
// visible. The load unit writes lane l's 16 bytes to LDS offset 16 l, and each lane chooses which 16 global
// bytes it fetches, so the tiles land in MFMA operand order: weight slot s holds, at 16 l, the 16 bytes lane l
// of the MFMA takes (row l % 16, k chunk l / 16); token block tb holds two 1 KB halves h = 0, 1 with, at 16 l,
// pair 16 tb + l % 16's k chunk 4 h + l / 16. Every operand read is one contiguous 1 KB ds_read_b128 per wave.
// Wave w computes 4 row blocks (MODE 0: gate slots 2 cg, 2 cg + 1 and their up slots, cg = w & 3, one FP8 group
// of 32 columns) for the 64 pairs of half w >> 2: 4 x 4 accumulators, 192 B of LDS reads per lane per k-step
// for 16 MFMAs. The operands of step k + 1 are read while the MFMAs of step k run; stage k is refilled with
// step k + PV_NS as soon as every wave has read it.
#define PV_NS 4
#define PV_A 0
#define PV_AS 16384
#define PV_B 17408
#define PV_BS 33792
#define PV_STAGE 34304
#ifndef PV_PP
#define PV_PP 1     // full groups run the ping-pong k-loop
#endif
#ifndef PV_CBW0
#define PV_CBW0 1   // column blocks per workgroup, w13 (MODE 0: 56 k-steps each at configs[3])
#endif
#ifndef PV_CBW1
#define PV_CBW1 2   // and w2 (MODE 1: 13 k-steps each)
#endif
typedef __attribute__((address_space(3))) void lds_void;
// Global-memory views for the epilogue stores inside the k-loop: through a generic pointer they would be FLAT stores,
// which count on the LDS counter too, and the compiler would then wait for every LDS-DMA step in flight before each
// operand read instead of only the one it needs.
typedef __attribute__((address_space(1))) uint32_t gmem_u32;
typedef __attribute__((address_space(1))) uint8_t gmem_u8;
typedef __attribute__((address_space(1))) v4f gmem_v4f;

__device__ __forceinline__ void wait_vm(int n) {   // s_waitcnt vmcnt(n), 0 <= n <= 20
#define PV_W(N) case N: __builtin_amdgcn_s_waitcnt(((N) & 15) | (7 << 4) | (15 << 8) | (((N) >> 4) << 14)); break;
    switch (n) {
        PV_W(1) PV_W(2) PV_W(3) PV_W(4) PV_W(5) PV_W(6) PV_W(7) PV_W(8) PV_W(9) PV_W(10)
        PV_W(11) PV_W(12) PV_W(13) PV_W(14) PV_W(15) PV_W(16) PV_W(17) PV_W(18) PV_W(19) PV_W(20)
        default: __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (15 << 8)); break;
    }
#undef PV_W
}

template <int N>
__device__ __forceinline__ void wait_vm_c() {   // s_waitcnt vmcnt(N), N a compile-time constant
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
template <int N>
struct IntC {
    static constexpr int value = N;
};

// Item L of the launch order (group, column blocks) on the 128-pair tile.
template <int MODE, int TILED>
__device__ __forceinline__ void prefill_item128(const PrefillArgs& a, const int L) {
    // more than one column block per workgroup (the epilogue inside the k-loop) or one (the epilogue after it)
    constexpr bool CBL = (MODE == 0 ? PV_CBW0 : PV_CBW1) > 1;
    extern __shared__ __align__(16) uint8_t smem[];   // PV_NS stages of PV_STAGE bytes
    __shared__ int s_row[PG_T];

    const int jx = L >> 3, gi = jx / a.n_it;
    const int g = item_group(a, gi * 8 + (L & 7)), cbi = jx - gi * a.n_it;
    if (g >= a.G || cbi >= a.n_it) return;
    // this workgroup's column blocks cb0 .. cb0 + ncb - 1 of group g, one after another through one k-pipeline
    const int cb0 = cbi * a.cbw, ncb = CBL ? min(a.cbw, a.n_cb - cb0) : 1;
    if (ncb <= 0) return;
    const int e = a.grp_expert[g];
    if (e < 0 || e >= a.E) return;
    const int p0 = min(max(a.grp_start[g], 0), a.n_pairs), m = min(min(a.grp_start[g + 1], a.n_pairs) - p0, PG_T);
    if (m <= 0) return;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cg = wave & 3, ph = wave >> 2;
    const int col = lane & 15, kb = lane >> 4;
    const int K = a.K, nk = K >> 7, Kh = K >> 1, Ks = K >> 5;
    const int I = a.N >> 1;
    // 16-row weight block of tile slot b = 0..15 in column block cb (MODE 0: slots 0-7 gate blocks, 8-15 the
    // matching up blocks); the next column block's blocks are PV_DNB further on
    auto block_of = [&](int b, int cb) {
        if (MODE == 0) return b < 8 ? (cb * 128 + 16 * b) >> 4 : (I + cb * 128 + 16 * (b - 8)) >> 4;
        return cb * 16 + b;
    };
    constexpr int PV_DNB = MODE == 0 ? 8 : 16;
    int slot_of[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) slot_of[j] = MODE == 0 ? (j < 2 ? 2 * cg + j : 8 + 2 * cg + (j - 2)) : 4 * cg + j;
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.W + (long long)e * a.stride_we, (uint32_t)a.stride_we);
    const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.S + (long long)e * a.stride_se, (uint32_t)a.stride_se);

    if (tid < PG_T) {
        const int p = p0 + (tid < m ? tid : 0);
        // MODE 1 without a table: input row = pair slot. A row outside the buffer becomes row x_rows, whose offsets
        // (xc_bytes, xs_bytes) are past both buffer descriptors, so its loads read zeros
        const int r = a.row_of_pair ? a.row_of_pair[p] : p;
        const int x_rows = (int)(a.xc_bytes / (uint32_t)a.ldx);
        s_row[tid] = (r >= 0 && r < x_rows) ? r : x_rows;
    }
    // the routing weights of this lane's pairs (MODE 0 epilogue), fetched now so the epilogue does not wait on them
    float wgt[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int pr = 64 * (wave >> 2) + 16 * u + (lane & 15);
        wgt[u] = MODE == 0 && pr < m ? a.wt_sorted[p0 + pr] : 0.f;
    }
    __syncthreads();

    // ---- DMA descriptors (MFMA A layout: lane l takes row l % 16, k chunk l / 16)
    const int nbw0 = block_of(2 * wave, cb0), nbw1 = block_of(2 * wave + 1, cb0);
    auto a_off = [&](int nb) {
        return TILED ? (uint32_t)(nb * nk * 1024 + col * 64 + kb * 16) : (uint32_t)((nb * 16 + col) * Kh + kb * 16);
    };
    const uint32_t a_voff0 = a_off(nbw0), a_voff1 = a_off(nbw1);
    const int a_ks = TILED ? 1024 : 64;
    const uint32_t a_cs = TILED ? (uint32_t)(PV_DNB * nk * 1024) : (uint32_t)(PV_DNB * 16 * Kh);   // per column block
    // weight scales of the 16 slots (64 bytes each per k-step). Tiled: a slot's 64 bytes are contiguous, so wave 0
    // fetches all 1 KB with 16 bytes per lane (lane l: slot l / 4, bytes 16 (l % 4)). Row-major: 4 bytes per row,
    // waves 0-3 fetch 4 slots each with 4 bytes per lane (lane l: slot 4 w + l / 16, row l % 16).
    const int asb = TILED ? block_of(lane >> 2, cb0) : block_of(4 * (wave & 3) + (lane >> 4), cb0), asr = lane & 15;
    const uint32_t as_voff = TILED ? (uint32_t)(asb * nk * 64 + (lane & 3) * 16) : (uint32_t)((asb * 16 + asr) * Ks);
    const int as_ks = TILED ? 64 : 4;
    const uint32_t as_cs = TILED ? (uint32_t)(PV_DNB * nk * 64) : (uint32_t)(PV_DNB * 16 * Ks);
    // MFMA B layout of token block `wave`: half h, lane l takes pair 16 wave + l % 16, k chunk 4 h + l / 16
    // activation rows through buffer descriptors too: reads past x_rows return 0, and with no FLAT-encoded load in
    // flight the compiler's waits on the LDS operand reads stay partial instead of draining all of them
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.xc, a.xc_bytes), xsr = buffer_rsrc(a.xs, a.xs_bytes);
    const uint32_t b0off = (uint32_t)s_row[16 * wave + col] * (uint32_t)a.ldx + kb * 16;
    const uint32_t bsoff = (uint32_t)s_row[(64 * (wave & 1) + lane) & (PG_T - 1)] * (uint32_t)a.ldxs;
    const bool ldb = 16 * wave < m;   // wave-uniform: the token block holds pairs of the group
    const bool lda = TILED ? wave == 0 : wave < 4, ldbs = (wave == 4 || wave == 5) && 64 * (wave & 1) < m;
    const int per_step = 2 + (lda ? 1 : 0) + (ldb ? 2 : 0) + (ldbs ? 1 : 0);
    // `full` (a compile-time flag inside the k-loop): the group holds all 128 pairs, so every wave loads its token
    // block and computes all four of its blocks, and the per-step checks of tb_on / ldb drop out
    // k-step kc of column block cb0 + c; aso / sso: its offsets into the expert's weights and scales (kc a_ks +
    // c a_cs, kc as_ks + c as_cs)
    auto issue = [&](uint32_t aso, uint32_t sso, int kc, int st, auto full_c) {
        uint8_t* so = smem + st * PV_STAGE;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(so + PV_A + 2 * wave * 1024), 16, a_voff0, aso, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(so + PV_A + (2 * wave + 1) * 1024), 16, a_voff1, aso, 0, 0);
        if (lda) {
            if (TILED) __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(so + PV_AS), 16, as_voff, sso, 0, 0);
            else __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(so + PV_AS + wave * 256), 4, as_voff, sso, 0, 0);
        }
        if (decltype(full_c)::value || ldb) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(so + PV_B + wave * 2048), 16, b0off, (uint32_t)(kc * 128), 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(so + PV_B + wave * 2048 + 1024), 16, b0off + 64, (uint32_t)(kc * 128), 0, 0);
        }
        if (ldbs)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xsr, (lds_void*)(so + PV_BS + (wave - 4) * 256), 4, bsoff, (uint32_t)(kc * 4), 0, 0);
    };

    // ---- operand registers (double-buffered) and their LDS reads
    const int lofs = lane * 16;
    bool tb_on[4];   // token blocks holding pairs (wave-uniform)
#pragma unroll
    for (int u = 0; u < 4; ++u) tb_on[u] = 64 * ph + 16 * u < m;
    v4i OA[2][4], OB0[2][4], OB1[2][4];
    uint32_t OSA[2], OSB[2];   // E8M0 bytes of the 4 weight slots / 4 token blocks, byte j each (MFMA byte select)
    // Every read of a step is issued before any is used: the token blocks unconditionally (a block without pairs reads
    // stale bytes of its slot, which no MFMA takes) and each E8M0 byte into a register of its own, packed after the
    // last read; a byte packed right behind its read would make each block wait for its own LDS round trip.
    auto read_ops = [&](int kk, int r, auto full_c) {
        constexpr bool full = decltype(full_c)::value;
        const uint8_t* st = smem + (kk % PV_NS) * PV_STAGE;
        if (full || tb_on[0]) {   // wave-uniform: a wave whose half of the group is empty runs no MFMA
            uint32_t ab[4], bb[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                OA[r][j] = *(const v4i*)(st + PV_A + slot_of[j] * 1024 + lofs);
                ab[j] = st[PV_AS + slot_of[j] * 64 + col * 4 + kb];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint8_t* bt = st + PV_B + (4 * ph + u) * 2048 + lofs;
                OB0[r][u] = *(const v4i*)bt;
                OB1[r][u] = *(const v4i*)(bt + 1024);
                bb[u] = st[PV_BS + (64 * ph + 16 * u + col) * 4 + kb];
            }
            OSA[r] = ab[0] | (ab[1] << 8) | (ab[2] << 16) | (ab[3] << 24);
            OSB[r] = bb[0] | (bb[1] << 8) | (bb[2] << 16) | (bb[3] << 24);
        }
    };
    v4f acc[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[j][u] = v4f{0.f, 0.f, 0.f, 0.f};
    auto mfmas = [&](int r, auto full_c) {
        constexpr bool full = decltype(full_c)::value;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (!full && !tb_on[u]) continue;
            const v8i bv = v8i{OB0[r][u].x, OB0[r][u].y, OB0[r][u].z, OB0[r][u].w, OB1[r][u].x, OB1[r][u].y, OB1[r][u].z, OB1[r][u].w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[j][u] = mfma_fp4w_fp8x_sel(j, u, v8i{OA[r][j].x, OA[r][j].y, OA[r][j].z, OA[r][j].w, 0, 0, 0, 0}, bv, acc[j][u], (int)OSA[r], (int)OSB[r]);
        }
    };
    // The tile of column block cb out of the accumulators: MODE 0 h = fq8(SwiGLU) of its 128 columns, MODE 1 the fp32
    // y2 rows; then the accumulators restart from zero for the next column block.
    auto epilogue = [&](int cb) __attribute__((always_inline)) {
        if (MODE == 0) {
            // acc[0..1][u]: gate rows of columns cb * 128 + 32 cg + 16 j + 4 kb + i (j = 0, 1); acc[2..3][u]: up rows
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (!tb_on[u]) continue;   // wave-uniform: no pair of this token block is in the group
                const int pr = 64 * ph + 16 * u + col;
                float h[2][4];
                float mx = 0.f;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float gv[4] = {acc[j][u].x, acc[j][u].y, acc[j][u].z, acc[j][u].w};
                    const float uv[4] = {acc[2 + j][u].x, acc[2 + j][u].y, acc[2 + j][u].z, acc[2 + j][u].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float gg = gv[i], uu = uv[i];
                        if (a.limit > 0.f) {
                            uu = fminf(fmaxf(uu, -a.limit), a.limit);
                            gg = fminf(gg, a.limit);
                        }
                        float hv = gg * (1.0f / (1.0f + expf(-gg))) * uu;
                        hv = bf16_round(hv * wgt[u]);
                        h[j][i] = hv;
                        mx = fmaxf(mx, fabsf(hv));
                    }
                }
                // the 32 columns of pair pr sit in the 4 lanes col + 16 kb: one FP8 group
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                const int ex = fq8_exponent(mx);
                if (pr < m) {
                    const long long p = p0 + pr;
                    const int c0 = cb * 128 + 32 * cg;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const uint32_t codes = fq8_code4_hw(h[j][0], h[j][1], h[j][2], h[j][3], ex);
                        *(gmem_u32*)(a.hc + p * a.ldhc + c0 + 16 * j + 4 * kb) = codes;
                    }
                    if (kb == 0) *(gmem_u8*)(a.hs + p * a.ldhs + (c0 >> 5)) = (uint8_t)(ex + 127);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int pr = 64 * ph + 16 * u + col;
                if (tb_on[u] && pr < m) {
                    // rows block_of(slot_of[j], cb) * 16 + 4 kb .. = cb * 256 + 64 cg + 16 j + 4 kb ..
                    float* o = a.y + (long long)(p0 + pr) * a.ldy + cb * 256 + 64 * cg + 4 * kb;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        gmem_v4f* q = (gmem_v4f*)(o + 16 * j);
                        if (MODE == 2) *q = *q + acc[j][u];   // the lo term's pass adds to the hi term's rows
                        else *q = acc[j][u];
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[j][u] = v4f{0.f, 0.f, 0.f, 0.f};
    };
    // The k-loop over the ncb x nk steps of this workgroup's column blocks (the DMA pipeline runs on across a column
    // block's end, so the next block's first steps are in flight during the epilogue), instantiated per value of this
    // wave's DMA count per step (2 .. 5, fixed for the item), so the steady-state wait below is one constant
    // s_waitcnt instead of a compare-and-branch tree on a runtime count.
    auto kloop = [&](auto ps_c, auto full_c) {
        constexpr int PS = decltype(ps_c)::value;
        const int T = ncb * nk;
        // step kk's data in LDS, visible to every wave. Issued before this point: steps 0 .. PV_NS - 1 (prologue)
        // and one refill per earlier sync, so the steps issued after kk number min(PV_NS - 1, T - 1) for kk = 0
        // and min(PV_NS - 2, T - 1 - kk) after that.
        auto sync_step = [&](int kk) {
            const int after = kk == 0 ? min(PV_NS - 1, T - 1) : min(PV_NS - 2, T - 1 - kk);
            if (after == PV_NS - 2) wait_vm_c<PS * (PV_NS - 2)>();
            else wait_vm(PS * after);
            __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0): own LDS reads done
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        };
        // the next step to issue (steps are issued in order): its k-step within the column block and its offsets
        int ikc = 0;
        uint32_t iao = 0, iso = 0;
        auto issue_next = [&](int st) {
            issue(iao, iso, ikc, st, full_c);
            iao += a_ks;
            iso += as_ks;
            if (++ikc == nk) {
                ikc = 0;
                iao += a_cs - (uint32_t)(nk * a_ks);
                iso += as_cs - (uint32_t)(nk * as_ks);
            }
        };
        int ekc = 0, ec = 0;   // column block and k-step of the next step whose MFMAs run
        auto step_done = [&]() {
            if constexpr (CBL) {
                if (++ekc == nk) { epilogue(cb0 + ec); ekc = 0; ++ec; }
            }
        };

        for (int s0 = 0; s0 < PV_NS; ++s0)
            if (s0 < T) issue_next(s0);
        sync_step(0);
        read_ops(0, 0, full_c);
        for (int kk = 0; kk < T; kk += 2) {
            if (kk + 1 < T) {
                sync_step(kk + 1);                                    // every wave has read step kk: refill its stage
                if (kk + PV_NS < T) issue_next(kk % PV_NS);
                read_ops(kk + 1, 1, full_c);
            }
            mfmas(0, full_c);
            step_done();
            if (kk + 1 >= T) break;
            if (kk + 2 < T) {
                sync_step(kk + 2);
                if (kk + 1 + PV_NS < T) issue_next((kk + 1) % PV_NS);
                read_ops(kk + 2, 0, full_c);
            }
            mfmas(1, full_c);
            step_done();
        }
    };
    // Full groups: a ping-pong k-loop. Waves 0-3 (pairs 0-63) and waves 4-7 (pairs 64-127) share the SIMDs pairwise
    // (wave w and w + 4 on SIMD w % 4) and would otherwise run their 16 MFMAs per step at the same time and their
    // DMA issue and operand reads at the same time. Here every step has two barriers, and waves 4-7 pass one barrier
    // before the loop, so their barrier j meets barrier j + 1 of waves 0-3: while one half runs step k's MFMAs, the
    // other half issues its DMA and reads step k's (or k + 1's) operands from LDS, and the matrix pipe of each SIMD
    // serves the two halves in turn. Data of step k is complete before either half reads it: waves 0-3 wait for
    // their own DMA of step k before their first barrier of step k, waves 4-7 for their DMA of step k + 1 before
    // their second barrier of step k (the one that releases waves 0-3 into step k + 1). A stage is refilled only
    // after both halves have read it (each half waits for its own LDS reads before its second barrier of the step).
    auto kloop_pp = [&](auto ps_c) {
        constexpr int PS = decltype(ps_c)::value;
        const int T = ncb * nk;
        const bool lag = ph == 1;   // wave-uniform
        int ikc = 0;
        uint32_t iao = 0, iso = 0;
        auto issue_next = [&](int st) {
            issue(iao, iso, ikc, st, IntC<1>{});
            iao += a_ks;
            iso += as_ks;
            if (++ikc == nk) {
                ikc = 0;
                iao += a_cs - (uint32_t)(nk * a_ks);
                iso += as_cs - (uint32_t)(nk * as_ks);
            }
        };
        int ekc = 0, ec = 0;
        auto step_done = [&]() {
            if constexpr (CBL) {
                if (++ekc == nk) { epilogue(cb0 + ec); ekc = 0; ++ec; }
            }
        };
        // own DMA of a step complete, with `after` later steps of this wave still in flight
        auto wait_own = [&](int after) {
            if (after == PV_NS - 2) wait_vm_c<PS * (PV_NS - 2)>();
            else wait_vm(PS * after);
        };
        auto barrier = [&]() {
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        };
        for (int s0 = 0; s0 < PV_NS - 1; ++s0)   // steps 0 .. PV_NS - 2; step k + PV_NS - 1 is issued in step k
            if (s0 < T) issue_next(s0);
        if (lag) {
            wait_own(min(PV_NS - 2, T - 1));     // own DMA of step 0
            barrier();                        // meets the first barrier of waves 0-3
        }
        for (int kk = 0; kk < T; ++kk) {
            if (!lag) wait_own(min(PV_NS - 2, T - 1 - kk));   // own DMA of step kk (steps up to kk + PV_NS - 2 issued)
            barrier();
            if (kk + PV_NS - 1 < T) issue_next((kk + PV_NS - 1) % PV_NS);   // the stage of step kk - 1: read by both halves
            read_ops(kk, 0, IntC<1>{});
            if (lag && kk + 1 < T) wait_own(min(PV_NS - 2, T - 2 - kk));   // own DMA of step kk + 1
            __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0): own LDS reads done
            barrier();
            mfmas(0, IntC<1>{});
            step_done();
        }
        if (!lag) barrier();                  // meets the last barrier of waves 4-7
    };
    // per_step = 2 (weight tiles) + 1 (weight scales: wave 0 tiled, waves 0-3 row-major) + 2 (a token block) + 1
    // (token scales: waves 4-5), never both scale streams in one wave: 2 .. 5; a full group loads every token
    // block (4 or 5)
    if (m == PG_T && PV_PP) {
        if (per_step == 4) kloop_pp(IntC<4>{});
        else kloop_pp(IntC<5>{});
    } else if (m == PG_T) {
        if (per_step == 4) kloop(IntC<4>{}, IntC<1>{});
        else kloop(IntC<5>{}, IntC<1>{});
    } else {
        switch (per_step) {
            case 2: kloop(IntC<2>{}, IntC<0>{}); break;
            case 3: kloop(IntC<3>{}, IntC<0>{}); break;
            case 4: kloop(IntC<4>{}, IntC<0>{}); break;
            default: kloop(IntC<5>{}, IntC<0>{}); break;
        }
    }
    if constexpr (!CBL) epilogue(cb0);   // one column block: the epilogue once, after the loop
}

template <int MODE, int TILED>
__global__ void __launch_bounds__(PG_THREADS) prefill_gemm_lds_kernel(const PrefillArgs a) {
    if (MODE == 2 && a.run_if && __builtin_amdgcn_readfirstlane(*a.run_if) == 0) return;
    prefill_item128<MODE, TILED>(a, (int)blockIdx.x);
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
    if (topk <= 8) {
        // the rows first, then every row's 16 bytes in flight at once (a loop over a runtime topk would wait for
        // each index before its row); summed in slot order as below
        int r[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) r[j] = j < topk ? inv[t * topk + j] : -1;
        v4f v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = r[j] >= 0 ? *(const v4f*)(y2 + (long long)r[j] * ldy2 + n) : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (r[j] >= 0) s += v[j];
    } else {
        for (int j = 0; j < topk; ++j) {
            const int r = inv[t * topk + j];   // -1: a pair the dispatch dropped (expert id outside [0, E))
            if (r >= 0) s += *(const v4f*)(y2 + (long long)r * ldy2 + n);
        }
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

// ------------------------------------------------------------------------------------------ 256-pair tiles
// The prefill path takes groups of up to 256 pairs (moe_dispatch tables with gmax 256) and a launch whose items pick
// their tile by the size of their group: groups of <= 128 pairs run the 128-pair tile above, larger ones a 256-row x
// 256-pair tile. Against two 128-pair items the large tile doubles the MFMAs per byte of weights loaded and halves
// how many groups (each re-reading its expert's weights) a popular expert takes. Wave w keeps the rows of the
// 128-pair tile (row quarter cg = w & 3: MODE 0 gate blocks 2 cg, 2 cg + 1 and their up blocks, MODE 1 row blocks
// 4 cg .. 4 cg + 3) for the 8 token blocks 2 u + ph of half ph = w >> 2 (alternate blocks, so both halves of every
// SIMD compute for any group size): 4 row blocks x 8 token blocks = 32 MFMAs per k-step, 128 accumulator registers,
// operands single-buffered. Stage (50 KB): weight slots 16 x 1 KB, their E8M0 bytes 16 x 64, token blocks 16 x 2 KB,
// the pairs' E8M0 words 256 x 4. Three stages: step k + 2 is issued in step k, into the stage of step k - 1. The
// k-loop is the ping-pong loop of the 128-pair tile (waves 4-7 one barrier behind waves 0-3).
#define P2_T 256
#define P2_NS 3
#define P2_A 0
#define P2_AS 16384
#define P2_B 17408
#define P2_BS 50176
#define P2_STAGE 51200

template <int MODE, int TILED>
__device__ __forceinline__ void prefill_item256(const PrefillArgs& a, const int L) {
    constexpr bool CBL = (MODE == 0 ? PV_CBW0 : PV_CBW1) > 1;
    extern __shared__ __align__(16) uint8_t smem[];   // P2_NS stages of P2_STAGE bytes
    __shared__ int s_row[P2_T];

    const int jx = L >> 3, gi = jx / a.n_it;
    const int g = item_group(a, gi * 8 + (L & 7)), cbi = jx - gi * a.n_it;
    if (g >= a.G || cbi >= a.n_it) return;
    const int cb0 = cbi * a.cbw, ncb = CBL ? min(a.cbw, a.n_cb - cb0) : 1;
    if (ncb <= 0) return;
    const int e = a.grp_expert[g];
    if (e < 0 || e >= a.E) return;
    const int p0 = min(max(a.grp_start[g], 0), a.n_pairs), m = min(min(a.grp_start[g + 1], a.n_pairs) - p0, P2_T);
    if (m <= 0) return;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cg = wave & 3, ph = wave >> 2;
    const int col = lane & 15, kb = lane >> 4;
    const int K = a.K, nk = K >> 7, Kh = K >> 1, Ks = K >> 5;
    const int I = a.N >> 1;
    auto block_of = [&](int b, int cb) {
        if (MODE == 0) return b < 8 ? (cb * 128 + 16 * b) >> 4 : (I + cb * 128 + 16 * (b - 8)) >> 4;
        return cb * 16 + b;
    };
    constexpr int PV_DNB = MODE == 0 ? 8 : 16;
    int slot_of[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) slot_of[j] = MODE == 0 ? (j < 2 ? 2 * cg + j : 8 + 2 * cg + (j - 2)) : 4 * cg + j;
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.W + (long long)e * a.stride_we, (uint32_t)a.stride_we);
    const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.S + (long long)e * a.stride_se, (uint32_t)a.stride_se);

    if (tid < P2_T) {
        const int p = p0 + (tid < m ? tid : 0);
        const int r = a.row_of_pair ? a.row_of_pair[p] : p;
        const int x_rows = (int)(a.xc_bytes / (uint32_t)a.ldx);
        s_row[tid] = (r >= 0 && r < x_rows) ? r : x_rows;
    }
    // the routing weights of this lane's pairs (MODE 0 epilogue), fetched now
    float wgt[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const int pr = 16 * (2 * u + ph) + col;
        wgt[u] = MODE == 0 && pr < m ? a.wt_sorted[p0 + pr] : 0.f;
    }
    __syncthreads();

    // ---- DMA descriptors: weight slots 2 w, 2 w + 1; token blocks 2 w, 2 w + 1 (two 1 KB halves each); weight scales
    // (tiled: wave 0, 16 B per lane; row-major: waves 0-3, 4 slots each); the pairs' E8M0 words (waves 4-7, 64 each)
    const int nbw0 = block_of(2 * wave, cb0), nbw1 = block_of(2 * wave + 1, cb0);
    auto a_off = [&](int nb) {
        return TILED ? (uint32_t)(nb * nk * 1024 + col * 64 + kb * 16) : (uint32_t)((nb * 16 + col) * Kh + kb * 16);
    };
    const uint32_t a_voff0 = a_off(nbw0), a_voff1 = a_off(nbw1);
    const int a_ks = TILED ? 1024 : 64;
    const uint32_t a_cs = TILED ? (uint32_t)(PV_DNB * nk * 1024) : (uint32_t)(PV_DNB * 16 * Kh);
    const int asb = TILED ? block_of(lane >> 2, cb0) : block_of(4 * (wave & 3) + (lane >> 4), cb0), asr = lane & 15;
    const uint32_t as_voff = TILED ? (uint32_t)(asb * nk * 64 + (lane & 3) * 16) : (uint32_t)((asb * 16 + asr) * Ks);
    const int as_ks = TILED ? 64 : 4;
    const uint32_t as_cs = TILED ? (uint32_t)(PV_DNB * nk * 64) : (uint32_t)(PV_DNB * 16 * Ks);
    const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.xc, a.xc_bytes), xsr = buffer_rsrc(a.xs, a.xs_bytes);
    const uint32_t b0off = (uint32_t)s_row[32 * wave + col] * (uint32_t)a.ldx + kb * 16;
    const uint32_t b1off = (uint32_t)s_row[32 * wave + 16 + col] * (uint32_t)a.ldx + kb * 16;
    const uint32_t bsoff = (uint32_t)s_row[(64 * (wave & 3) + lane) & (P2_T - 1)] * (uint32_t)a.ldxs;
    const bool ldb0 = 32 * wave < m, ldb1 = 32 * wave + 16 < m;   // wave-uniform: the token block holds pairs
    const bool lda = TILED ? wave == 0 : wave < 4, ldbs = wave >= 4 && 64 * (wave - 4) < m;
    const int per_step = 2 + (lda ? 1 : 0) + (ldb0 ? 2 : 0) + (ldb1 ? 2 : 0) + (ldbs ? 1 : 0);

    const int lofs = lane * 16;
    bool tb_on[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) tb_on[u] = 16 * (2 * u + ph) < m;
    const bool any_on = tb_on[0];
    v4i OA[4], OB0[8], OB1[8];
    uint32_t OSA, OSB[2];
    // per-lane LDS offsets within a stage: weight slots relative to slot_of[0], token blocks of this half, scales
    const uint32_t lofs_a = (uint32_t)(P2_A + slot_of[0] * 1024 + lofs), lofs_b = (uint32_t)(P2_B + ph * 2048 + lofs);
    const uint32_t lofs_as = (uint32_t)(P2_AS + slot_of[0] * 64 + col * 4 + kb), lofs_bs = (uint32_t)(P2_BS + 16 * ph * 4 + col * 4 + kb);
    // Every read of a step is issued before any of them is used: the token blocks unconditionally (a block without
    // pairs reads stale bytes of its slot, which no MFMA takes) and each E8M0 byte into a register of its own, packed
    // after the last read. (Packing each byte right behind its read made every block wait for its own LDS round trip:
    // eight serial round trips per step, the longest part of the step.)
    auto read_ops = [&](int st) {
        const uint32_t so = (uint32_t)st * P2_STAGE;
        const uint32_t oa = lofs_a + so, ob = lofs_b + so, osa = lofs_as + so, osb = lofs_bs + so;
        uint32_t ab[4], bb[8];
        if (any_on) {   // wave-uniform: a wave whose half of the group is empty reads and computes nothing
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int dj = MODE == 0 ? (j < 2 ? j : 8 + (j - 2)) : j;   // slot_of[j] - slot_of[0]
                OA[j] = *(const v4i*)(smem + oa + dj * 1024);
                ab[j] = smem[osa + dj * 64];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                OB0[u] = *(const v4i*)(smem + ob + u * 4096);
                OB1[u] = *(const v4i*)(smem + ob + u * 4096 + 1024);
                bb[u] = smem[osb + u * 128];
            }
            OSA = ab[0] | (ab[1] << 8) | (ab[2] << 16) | (ab[3] << 24);
            OSB[0] = bb[0] | (bb[1] << 8) | (bb[2] << 16) | (bb[3] << 24);
            OSB[1] = bb[4] | (bb[5] << 8) | (bb[6] << 16) | (bb[7] << 24);
        }
    };
    v4f acc[4][8];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[j][u] = v4f{0.f, 0.f, 0.f, 0.f};
    auto mfmas = [&]() {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (!tb_on[u]) continue;
            const v8i bv = v8i{OB0[u].x, OB0[u].y, OB0[u].z, OB0[u].w, OB1[u].x, OB1[u].y, OB1[u].z, OB1[u].w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[j][u] = mfma_fp4w_fp8x_sel(j, u & 3, v8i{OA[j].x, OA[j].y, OA[j].z, OA[j].w, 0, 0, 0, 0}, bv, acc[j][u], (int)OSA,
                                               (int)OSB[u >> 2]);
        }
    };
    auto epilogue = [&](int cb) __attribute__((always_inline)) {
        if (MODE == 0) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (!tb_on[u]) continue;
                const int pr = 16 * (2 * u + ph) + col;
                float h[2][4];
                float mx = 0.f;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float gv[4] = {acc[j][u].x, acc[j][u].y, acc[j][u].z, acc[j][u].w};
                    const float uv[4] = {acc[2 + j][u].x, acc[2 + j][u].y, acc[2 + j][u].z, acc[2 + j][u].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        float gg = gv[i], uu = uv[i];
                        if (a.limit > 0.f) {
                            uu = fminf(fmaxf(uu, -a.limit), a.limit);
                            gg = fminf(gg, a.limit);
                        }
                        float hv = gg * (1.0f / (1.0f + expf(-gg))) * uu;
                        hv = bf16_round(hv * wgt[u]);
                        h[j][i] = hv;
                        mx = fmaxf(mx, fabsf(hv));
                    }
                }
                mx = fmaxf(mx, __shfl_xor(mx, 16));
                mx = fmaxf(mx, __shfl_xor(mx, 32));
                const int ex = fq8_exponent(mx);
                if (pr < m) {
                    const long long p = p0 + pr;
                    const int c0 = cb * 128 + 32 * cg;
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const uint32_t codes = fq8_code4_hw(h[j][0], h[j][1], h[j][2], h[j][3], ex);
                        *(gmem_u32*)(a.hc + p * a.ldhc + c0 + 16 * j + 4 * kb) = codes;
                    }
                    if (kb == 0) *(gmem_u8*)(a.hs + p * a.ldhs + (c0 >> 5)) = (uint8_t)(ex + 127);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int pr = 16 * (2 * u + ph) + col;
                if (tb_on[u] && pr < m) {
                    float* o = a.y + (long long)(p0 + pr) * a.ldy + cb * 256 + 64 * cg + 4 * kb;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        gmem_v4f* q = (gmem_v4f*)(o + 16 * j);
                        if (MODE == 2) *q = *q + acc[j][u];   // the lo term's pass adds to the hi term's rows
                        else *q = acc[j][u];
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int u = 0; u < 8; ++u) acc[j][u] = v4f{0.f, 0.f, 0.f, 0.f};
    };
    // The ping-pong k-loop over the ncb x nk steps with three stages: in step k, after its first barrier, the stage of
    // step k - 1 (read by both halves by then) takes step k + 2. Instantiated per wave DMA count (2 .. 8), so the
    // waits are constants.
    auto kloop = [&](auto ps_c) {
        constexpr int PS = decltype(ps_c)::value;
        const int T = ncb * nk;
        const bool lag = ph == 1;
        uint32_t iao = 0, iso = 0, ixo = 0;
        int ikc = 0;
        auto issue_st = [&](int st) {
            uint8_t* so = smem + st * P2_STAGE;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(so + P2_A + 2 * wave * 1024), 16, a_voff0, iao, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(wr, (lds_void*)(so + P2_A + (2 * wave + 1) * 1024), 16, a_voff1, iao, 0, 0);
            if (lda) {
                if (TILED) __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(so + P2_AS), 16, as_voff, iso, 0, 0);
                else __builtin_amdgcn_raw_ptr_buffer_load_lds(sr, (lds_void*)(so + P2_AS + wave * 256), 4, as_voff, iso, 0, 0);
            }
            if (ldb0) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(so + P2_B + 2 * wave * 2048), 16, b0off, ixo, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(so + P2_B + 2 * wave * 2048 + 1024), 16, b0off + 64, ixo, 0, 0);
            }
            if (ldb1) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(so + P2_B + (2 * wave + 1) * 2048), 16, b1off, ixo, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (lds_void*)(so + P2_B + (2 * wave + 1) * 2048 + 1024), 16, b1off + 64, ixo, 0, 0);
            }
            if (ldbs)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xsr, (lds_void*)(so + P2_BS + (wave - 4) * 256), 4, bsoff, ixo >> 5, 0, 0);
            iao += a_ks;
            iso += as_ks;
            ixo += 128;
            if constexpr (CBL) {
                if (++ikc == nk) {
                    ikc = 0;
                    ixo = 0;
                    iao += a_cs - (uint32_t)(nk * a_ks);
                    iso += as_cs - (uint32_t)(nk * as_ks);
                }
            }
        };
        int ekc = 0, ec = 0;
        auto step_done = [&]() {
            if constexpr (CBL) {
                if (++ekc == nk) { epilogue(cb0 + ec); ekc = 0; ++ec; }
            }
        };
        auto barrier = [&]() {
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        };
        // one k-step in stage st; ISS: it refills the stage of step k - 1 with step k + 2; WA / WB: later steps of this
        // wave in flight when it waits for its DMA of this step (before the first barrier) and of the next (before
        // the second; WB < 0: no wait). Both halves take both waits.
        auto step = [&](int st, auto iss_c, auto wa_c, auto wb_c) {
            constexpr int WA = decltype(wa_c)::value, WB = decltype(wb_c)::value;
            wait_vm_c<PS * WA>();
            barrier();
            read_ops(st);
            if constexpr (decltype(iss_c)::value != 0) issue_st(st == 0 ? 2 : st - 1);
            if constexpr (WB >= 0) wait_vm_c<PS * WB>();
            __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));   // lgkmcnt(0): own LDS reads done
            barrier();
            mfmas();
            step_done();
        };
        issue_st(0);   // steps 0, 1 (T >= PG_PF = 3)
        issue_st(1);
        if (lag) {
            wait_vm_c<PS * 1>();              // own DMA of step 0
            barrier();                        // meets the first barrier of waves 0-3
        }
        // steady state: steps 0 .. T - 3, each refilling and waiting with one later step in flight; then T - 2, T - 1
        int st = 0;
        for (int kk = 0; kk < T - 2; ++kk) {
            step(st, IntC<1>{}, IntC<1>{}, IntC<1>{});
            st = st == P2_NS - 1 ? 0 : st + 1;
        }
        step(st, IntC<0>{}, IntC<1>{}, IntC<0>{});
        st = st == P2_NS - 1 ? 0 : st + 1;
        step(st, IntC<0>{}, IntC<0>{}, IntC<-1>{});
        if (!lag) barrier();                  // meets the last barrier of waves 4-7
    };
    switch (per_step) {
        case 2: kloop(IntC<2>{}); break;
        case 3: kloop(IntC<3>{}); break;
        case 4: kloop(IntC<4>{}); break;
        case 5: kloop(IntC<5>{}); break;
        case 6: kloop(IntC<6>{}); break;
        case 7: kloop(IntC<7>{}); break;
        default: kloop(IntC<8>{}); break;
    }
    if constexpr (!CBL) epilogue(cb0);
}


// The prefill path's launch: each item takes the 256-pair tile when its group holds more than 128 pairs.
template <int MODE, int TILED>
__global__ void __launch_bounds__(PG_THREADS) prefill_gemm_mixed_kernel(const PrefillArgs a) {
    if (MODE == 2 && a.run_if && __builtin_amdgcn_readfirstlane(*a.run_if) == 0) return;
    const int L = (int)blockIdx.x;
    const int jx = L >> 3, g = item_group(a, (jx / a.n_it) * 8 + (L & 7));
    if (g >= a.G) return;
    const int p0 = min(max(a.grp_start[g], 0), a.n_pairs), m = min(a.grp_start[g + 1], a.n_pairs) - p0;
    if (m > PG_T) prefill_item256<MODE, TILED>(a, L);
    else prefill_item128<MODE, TILED>(a, L);
}

// mixed: groups of <= 256 pairs (the prefill path's launch); otherwise <= 128 (the 128-pair tile alone)
static int launch_prefill(PrefillArgs& a, int mode, int tiled, bool mixed, hipStream_t st) {
    a.g_pad = (a.G + 7) & ~7;
    a.cbw = (mode == 0 || a.K >= 4096) ? PV_CBW0 : PV_CBW1;   // long k-loops: one column block per workgroup
    a.n_it = (a.n_cb + a.cbw - 1) / a.cbw;
    const long long items = (long long)a.n_it * a.g_pad;   // a multiple of 8
    if (items > 0x7FFFFFFFll) return DSV41_EINVAL;
    const dim3 grid((unsigned)items), block(PG_THREADS);
    const size_t lds = mixed ? (size_t)max(PV_NS * PV_STAGE, P2_NS * P2_STAGE) : (size_t)PV_NS * PV_STAGE;
#define PV_LAUNCH(K, M, T)                                                                                            \
    do {                                                                                                          \
        const hipError_t err = hipFuncSetAttribute((const void*)K<M, T>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                                   (int)lds);                                                     \
        if (err != hipSuccess) return (int)err;                                                                   \
        K<M, T><<<grid, block, lds, st>>>(a);                                                                     \
    } while (0)
    if (mixed) {
        if (mode == 0) { if (tiled) PV_LAUNCH(prefill_gemm_mixed_kernel, 0, 1); else PV_LAUNCH(prefill_gemm_mixed_kernel, 0, 0); }
        else if (mode == 1) { if (tiled) PV_LAUNCH(prefill_gemm_mixed_kernel, 1, 1); else PV_LAUNCH(prefill_gemm_mixed_kernel, 1, 0); }
        else { if (tiled) PV_LAUNCH(prefill_gemm_mixed_kernel, 2, 1); else PV_LAUNCH(prefill_gemm_mixed_kernel, 2, 0); }
    } else {
        if (mode == 0) { if (tiled) PV_LAUNCH(prefill_gemm_lds_kernel, 0, 1); else PV_LAUNCH(prefill_gemm_lds_kernel, 0, 0); }
        else if (mode == 1) { if (tiled) PV_LAUNCH(prefill_gemm_lds_kernel, 1, 1); else PV_LAUNCH(prefill_gemm_lds_kernel, 1, 0); }
        else { if (tiled) PV_LAUNCH(prefill_gemm_lds_kernel, 2, 1); else PV_LAUNCH(prefill_gemm_lds_kernel, 2, 0); }
    }
#undef PV_LAUNCH
    return (int)hipGetLastError();
}

extern "C" int dsv41_prefill_up(const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, int x_rows, const uint8_t* W13, long long stride_we,
                                const uint8_t* S13, long long stride_se, int tiled, int E, int H, int I, const int* grp_expert,
                                const int* grp_start, int G, const int* tok_sorted, const float* wt_sorted, float limit, uint8_t* hc,
                                long long ldhc, uint8_t* hs, long long ldhs, const int* grp_order, void* stream) {
    if (!xc || !xs || !W13 || !S13 || !grp_expert || !grp_start || !tok_sorted || !wt_sorted || !hc || !hs) return DSV41_EINVAL;
    if (x_rows < 1 || (long long)x_rows * ldx > 0xFFFFFFFFll || (long long)x_rows * ldxs > 0xFFFFFFFFll) return DSV41_EINVAL;
    if (E < 1 || H < 128 * PG_PF || (H & 127) || I <= 0 || (I & 127) || G < 0 || ldx < H || (ldx & 15) || (((uintptr_t)xc) & 15) || ldxs < H / 32 ||
        (ldxs & 3) || (((uintptr_t)xs) & 3) || ldhc < I || (ldhc & 3) || (((uintptr_t)hc) & 3) || ldhs < I / 32)
        return DSV41_EINVAL;
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll || stride_we < (long long)2 * I * (H / 2) ||
        stride_se < (long long)2 * I * (H / 32))
        return DSV41_EINVAL;
    if (G == 0) return 0;
    PrefillArgs a{xc, ldx, xs, ldxs, (uint32_t)(x_rows * ldx), (uint32_t)(x_rows * ldxs), W13, stride_we, S13, stride_se, 2 * I, H, E,
                  grp_expert, grp_start, G, tok_sorted, wt_sorted, limit, hc, ldhc, hs, ldhs, nullptr, 0, I / 128, 0, 0x7FFFFFFF};
    a.grp_order = grp_order;
    return launch_prefill(a, 0, tiled, true, (hipStream_t)stream);
}

extern "C" int dsv41_prefill_down(const uint8_t* hc, long long ldhc, const uint8_t* hs, long long ldhs, int h_rows, const uint8_t* W2, long long stride_we,
                                  const uint8_t* S2, long long stride_se, int tiled, int E, int H, int I, const int* grp_expert,
                                  const int* grp_start, int G, float* y2, long long ldy, const int* grp_order, void* stream) {
    if (!hc || !hs || !W2 || !S2 || !grp_expert || !grp_start || !y2) return DSV41_EINVAL;
    if (h_rows < 1 || (long long)h_rows * ldhc > 0xFFFFFFFFll || (long long)h_rows * ldhs > 0xFFFFFFFFll) return DSV41_EINVAL;
    if (E < 1 || H <= 0 || (H & 255) || I < 128 * PG_PF || (I & 127) || G < 0 || ldhc < I || (ldhc & 15) || (((uintptr_t)hc) & 15) || ldhs < I / 32 ||
        (ldhs & 3) || (((uintptr_t)hs) & 3) || ldy < H || (ldy & 3) || (((uintptr_t)y2) & 15))
        return DSV41_EINVAL;
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll || stride_we < (long long)H * (I / 2) ||
        stride_se < (long long)H * (I / 32))
        return DSV41_EINVAL;
    if (G == 0) return 0;
    PrefillArgs a{hc, ldhc, hs, ldhs, (uint32_t)(h_rows * ldhc), (uint32_t)(h_rows * ldhs), W2, stride_we, S2, stride_se, H, I, E,
                  grp_expert, grp_start, G, nullptr, nullptr, 0.f, nullptr, 0, nullptr, 0, y2, ldy, H / 256, 0, h_rows};
    a.grp_order = grp_order;
    return launch_prefill(a, 1, tiled, true, (hipStream_t)stream);
}

// The groups of a dispatch ordered by pair count, largest first (a counting sort over the counts 0 .. 256 in one
// workgroup; groups without an expert in the table (-1) count 0, and counts above 256 count 256, as the tile kernels
// compute at most 256 pairs of a group). Within one count the order is whatever the LDS atomics give: the prefill
// launches write disjoint rows per item, so their results do not depend on it.
__global__ void __launch_bounds__(1024) group_order_kernel(const int* __restrict__ grp_expert, const int* __restrict__ grp_start, int G,
                                                           int n_pairs, int* __restrict__ order) {
    __shared__ int s_bin[258];
    const int tid = threadIdx.x;
    for (int i = tid; i < 258; i += 1024) s_bin[i] = 0;
    __syncthreads();
    auto bin_of = [&](int g) {   // 0 for 256 pairs .. 256 for none
        if (grp_expert[g] < 0) return 256;
        const int p0 = min(max(grp_start[g], 0), n_pairs), p1 = min(max(grp_start[g + 1], p0), n_pairs);
        return 256 - min(p1 - p0, 256);
    };
    for (int g = tid; g < G; g += 1024) atomicAdd(&s_bin[bin_of(g)], 1);
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int b = 0; b < 257; ++b) {
            const int c = s_bin[b];
            s_bin[b] = run;
            run += c;
        }
    }
    __syncthreads();
    for (int g = tid; g < G; g += 1024) order[atomicAdd(&s_bin[bin_of(g)], 1)] = g;
}

extern "C" int dsv41_group_order(const int* grp_expert, const int* grp_start, int G, int n_pairs, int* order, void* stream) {
    if (!grp_expert || !grp_start || !order || G < 0 || n_pairs < 0) return DSV41_EINVAL;
    if (G == 0) return 0;
    group_order_kernel<<<1, 1024, 0, (hipStream_t)stream>>>(grp_expert, grp_start, G, n_pairs, order);
    return (int)hipGetLastError();
}

// The second FP8 term of off-grid activations (xlc / xls / lo_flag of dsv41_quant_fp8_split, all or none): checked like
// the first, then run as a MODE 2 pass over the same groups that adds into the rows the first pass wrote.
static bool lo_term_bad(const uint8_t* xc, const uint8_t* xlc, const uint8_t* xls, const int* lo_flag) {
    return (xlc != nullptr) != (xls != nullptr) || (lo_flag && !xlc) || (((uintptr_t)xlc) & 15) || (((uintptr_t)xls) & 3) ||
           (xlc && xlc == xc);
}

static int lo_pass(const PrefillArgs& a, const uint8_t* xlc, const uint8_t* xls, const int* lo_flag, int tiled, bool mixed, hipStream_t st) {
    if (!xlc) return 0;
    PrefillArgs b = a;
    b.xc = xlc;
    b.xs = xls;
    b.run_if = lo_flag;
    return launch_prefill(b, 2, tiled, mixed, st);
}

extern "C" int dsv41_fp4_grouped_gemm_t128(const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, int x_rows,
                                           const uint8_t* xlc, const uint8_t* xls, const int* lo_flag, const int* row_of_pair,
                                           const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled, int E, int N,
                                           int K, const int* grp_expert, const int* grp_start, int G, int n_pairs, float* y, long long ldy,
                                           void* stream) {
    if (!xc || !xs || !W || !S || !grp_expert || !grp_start || !y || n_pairs < 0) return DSV41_EINVAL;
    if (lo_term_bad(xc, xlc, xls, lo_flag)) return DSV41_EINVAL;
    if (!row_of_pair && n_pairs > x_rows) return DSV41_EINVAL;   // without a table, pair p reads input row p
    if (x_rows < 1 || (long long)x_rows * ldx > 0xFFFFFFFFll || (long long)x_rows * ldxs > 0xFFFFFFFFll) return DSV41_EINVAL;
    if (E < 1 || N <= 0 || (N & 255) || K < 128 * PG_PF || (K & 127) || G < 0 || ldx < K || (ldx & 15) || (((uintptr_t)xc) & 15) ||
        ldxs < K / 32 || (ldxs & 3) || (((uintptr_t)xs) & 3) || ldy < N || (ldy & 3) || (((uintptr_t)y) & 15))
        return DSV41_EINVAL;
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll || stride_we < (long long)N * (K / 2) ||
        stride_se < (long long)N * (K / 32))
        return DSV41_EINVAL;
    if (G == 0) return 0;
    PrefillArgs a{xc, ldx, xs, ldxs, (uint32_t)(x_rows * ldx), (uint32_t)(x_rows * ldxs), W, stride_we, S, stride_se, N, K, E,
                  grp_expert, grp_start, G, row_of_pair, nullptr, 0.f, nullptr, 0, nullptr, 0, y, ldy, N / 256, 0, n_pairs};
    const int rc = launch_prefill(a, 1, tiled, false, (hipStream_t)stream);
    return rc ? rc : lo_pass(a, xlc, xls, lo_flag, tiled, false, (hipStream_t)stream);
}

// out[row_out[p]] (+)= fl(wt[p] * y2[p]) for the pairs of every group g with an expert in [0, E) (its first P2_T pairs,
// those the tile kernels computed), one workgroup per (1024 columns, group, SCAT_ROWS pairs), pairs in slot order. sm: 0
// store, 1 read, add and write (the output rows are distinct, so no two workgroups touch one element), 2 fp32 atomic
// adds.
#define SCAT_UNROLL 8
#define SCAT_ROWS 32
__global__ void __launch_bounds__(256) scatter_rows_kernel(const float* __restrict__ y2, long long ldy2, const int* __restrict__ grp_expert,
                                                           const int* __restrict__ grp_start, int E, int n_pairs,
                                                           const int* __restrict__ row_out, const float* __restrict__ wt,
                                                           const int* __restrict__ distinct, int accum, float* out, long long ldo,
                                                           int out_rows, int N) {
    const int g = blockIdx.y;
    const int e = grp_expert[g];
    if (e < 0 || e >= E) return;
    const int gp0 = min(max(grp_start[g], 0), n_pairs), gp1 = min(min(grp_start[g + 1], n_pairs), gp0 + P2_T);
    const int p0 = gp0 + (int)blockIdx.z * SCAT_ROWS, p1 = min(gp1, p0 + SCAT_ROWS);
    const int c = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (c >= N || p1 <= p0) return;
    const int d = distinct ? __builtin_amdgcn_readfirstlane(*distinct) : 0;
    const int sm = d ? (accum ? 1 : 0) : 2;
    for (int q = p0; q < p1; q += SCAT_UNROLL) {
        v4f v[SCAT_UNROLL];
        int r[SCAT_UNROLL];
        float w[SCAT_UNROLL];
#pragma unroll
        for (int i = 0; i < SCAT_UNROLL; ++i) {   // every load of the batch in flight before the first write
            const int p = min(q + i, p1 - 1);
            r[i] = q + i < p1 ? row_out[p] : -1;
            w[i] = wt[p];
            v[i] = *(const v4f*)(y2 + (long long)p * ldy2 + c);
        }
#pragma unroll
        for (int i = 0; i < SCAT_UNROLL; ++i) {
            if ((unsigned)r[i] >= (unsigned)out_rows) continue;
            float* o = out + (long long)r[i] * ldo + c;
            const v4f pv = v4f{__fmul_rn(v[i].x, w[i]), __fmul_rn(v[i].y, w[i]), __fmul_rn(v[i].z, w[i]), __fmul_rn(v[i].w, w[i])};
            if (sm == 0) {
                *(v4f*)o = pv;
            } else if (sm == 1) {
                const v4f ov = *(const v4f*)o;
                *(v4f*)o = v4f{__fadd_rn(ov.x, pv.x), __fadd_rn(ov.y, pv.y), __fadd_rn(ov.z, pv.z), __fadd_rn(ov.w, pv.w)};
            } else {
                unsafeAtomicAdd(o, pv.x);
                unsafeAtomicAdd(o + 1, pv.y);
                unsafeAtomicAdd(o + 2, pv.z);
                unsafeAtomicAdd(o + 3, pv.w);
            }
        }
    }
}

// The reference's grouped GEMM with its weighted output-row epilogue (moe_kernels.py:29-80, 155-200): y2[p] = codes(x)
// [row] . deq(W[e_g])^T on the mixed 128 / 256-pair tile kernel (groups of up to 256 pairs), then out[row_out[p]] +=
// fl(wt[p] * y2[p]) in a second launch (an epilogue of that form inside the tile kernel's k-loop made its compiled loop
// twice as slow).
extern "C" int dsv41_fp4_grouped_gemm_scatter(const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, int x_rows,
                                              const uint8_t* xlc, const uint8_t* xls, const int* lo_flag,
                                              const int* row_of_pair, const uint8_t* W, long long stride_we, const uint8_t* S,
                                              long long stride_se, int tiled, int E, int N, int K, const int* grp_expert, const int* grp_start,
                                              int G, int n_pairs, const int* row_out, const float* wt, const int* distinct, int accum,
                                              float* out, long long ldo, int out_rows, float* y2, long long ldy2, void* stream) {
    if (!xc || !xs || !W || !S || !grp_expert || !grp_start || !row_out || !wt || !out || !y2 || n_pairs < 0 || out_rows < 0 || accum < 0 ||
        accum > 1)
        return DSV41_EINVAL;
    if (lo_term_bad(xc, xlc, xls, lo_flag)) return DSV41_EINVAL;
    if (!row_of_pair && n_pairs > x_rows) return DSV41_EINVAL;   // without a table, pair p reads input row p
    if (x_rows < 1 || (long long)x_rows * ldx > 0xFFFFFFFFll || (long long)x_rows * ldxs > 0xFFFFFFFFll) return DSV41_EINVAL;
    if (E < 1 || N <= 0 || (N & 255) || K < 128 * PG_PF || (K & 127) || G < 0 || G > 0xFFFF || ldx < K || (ldx & 15) || (((uintptr_t)xc) & 15) ||
        ldxs < K / 32 || (ldxs & 3) || (((uintptr_t)xs) & 3) || ldo < N || (ldo & 3) || (((uintptr_t)out) & 15) || ldy2 < N || (ldy2 & 3) ||
        (((uintptr_t)y2) & 15))
        return DSV41_EINVAL;
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll || stride_we < (long long)N * (K / 2) ||
        stride_se < (long long)N * (K / 32))
        return DSV41_EINVAL;
    if (G == 0 || n_pairs == 0 || out_rows == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    PrefillArgs a{xc, ldx, xs, ldxs, (uint32_t)(x_rows * ldx), (uint32_t)(x_rows * ldxs), W, stride_we, S, stride_se, N, K, E,
                  grp_expert, grp_start, G, row_of_pair, nullptr, 0.f, nullptr, 0, nullptr, 0, y2, ldy2, N / 256, 0, n_pairs};
    int rc = launch_prefill(a, 1, tiled, true, st);
    if (rc == 0) rc = lo_pass(a, xlc, xls, lo_flag, tiled, true, st);
    if (rc != 0) return rc;
    const dim3 grid((unsigned)((N + 1023) / 1024), (unsigned)G, P2_T / SCAT_ROWS);
    scatter_rows_kernel<<<grid, 256, 0, st>>>(y2, ldy2, grp_expert, grp_start, E, n_pairs, row_out, wt, distinct, accum, out, ldo, out_rows, N);
    return (int)hipGetLastError();
}

// One workgroup: a bitmap of the output rows in LDS, set by the first n_placed (or n) entries of row_out; an entry whose
// bit was already set is a repeated row. Rows outside [0, out_rows) are never written, so they are not counted.
// unchecked: out_rows exceeds the bitmap; the flag is 0 (the atomic form).
__global__ void __launch_bounds__(1024) rows_distinct_kernel(const int* __restrict__ row_out, int n, const int* __restrict__ n_placed,
                                                             int out_rows, int unchecked, int* flag) {
    extern __shared__ unsigned bits[];
    __shared__ int s_dup;
    if (unchecked) {
        if (threadIdx.x == 0) flag[0] = 0;
        return;
    }
    const int nw = (out_rows + 31) >> 5;
    for (int i = threadIdx.x; i < nw; i += blockDim.x) bits[i] = 0u;
    if (threadIdx.x == 0) s_dup = 0;
    __syncthreads();
    const int cnt = n_placed ? min(max(*n_placed, 0), n) : n;
    for (int p = threadIdx.x; p < cnt; p += blockDim.x) {
        const int r = row_out[p];
        if ((unsigned)r < (unsigned)out_rows) {
            const unsigned m = 1u << (r & 31);
            if (atomicOr(&bits[r >> 5], m) & m) s_dup = 1;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) flag[0] = s_dup ? 0 : 1;
}

#define DISTINCT_MAX_ROWS (1 << 20)   // 128 KiB of bitmap

// GroupedPairs' distinct-rows flag for dsv41_fp4_grouped_gemm_scatter: *flag = 1 when no two of the first n_placed
// (device int; NULL: n) entries of row_out inside [0, out_rows) are equal, else 0 (also for out_rows beyond the bitmap).
extern "C" int dsv41_rows_distinct(const int* row_out, int n, const int* n_placed, int out_rows, int* flag, void* stream) {
    if (!row_out || !flag || n < 0 || out_rows < 0) return DSV41_EINVAL;
    hipStream_t st = (hipStream_t)stream;
    const int unchecked = out_rows > DISTINCT_MAX_ROWS ? 1 : 0;
    const size_t lds = unchecked ? 4 : (size_t)max((out_rows + 31) >> 5, 1) * 4;
    const hipError_t err = hipFuncSetAttribute((const void*)rows_distinct_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) return (int)err;
    rows_distinct_kernel<<<1, 1024, lds, st>>>(row_out, n, n_placed, out_rows, unchecked, flag);
    return (int)hipGetLastError();
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
