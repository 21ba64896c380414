// Decode up projection of one MoE layer (M <= 16 tokens) as ONE kernel with no cross-workgroup communication:
// routing, expert bucketing, activation quantisation, the w13 grouped GEMV and the SwiGLU epilogue.
//
// Workgroup (column block cb, group slot g) owns the 32 SwiGLU columns c0 = 32 cb .. c0 + 31 of the g-th selected
// expert: gate rows c0..c0+31 and up rows I + c0 .. I + c0 + 31 of W13 over the full K, as 4 row blocks of 16 x 2
// K-halves = 8 waves (all streaming 1 KiB weight tiles). Because the workgroup holds complete gate and up values
// of one FP8 group (32 columns), it produces h = fq8(bf16(w * silu(min(g, L)) * clamp(u, +-L))) itself
// (fused.py:284-306, routing weight folded in before rounding, fused.py:297-302): gate/up never leave the chip.
//
// Every workgroup recomputes the routing (one wave per token: fused2.gate_topk, fused2.py:418-452) and the
// bucketing (stable: experts ascending, tokens ascending inside an expert; cukern.moe_dispatch semantics,
// p2p.cu:90-132) from the logits; workgroup (0, 0) publishes the routing and the tables for the down projection.
// The reference runs these steps as gate_topk + moe_dispatch + fp4_gemm_tc(w13) + swiglu_quant launches
// (decode.py:316-335, 354-358).
#include "common.h"
#include "gate.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define UP_WAVES 8
#define UP_MAXM 16
#define UP_MAXK 16
#define UP_MAXE 512
#define UP_WSC 2048   // SCL: E8M0 bytes of a wave's weight stream staged in LDS (<= 32 k-chunks of 64 bytes)

struct DecodeUpArgs {
    const float* logits; long long ldl;      // fp32 [M][E] router logits (or NULL: eid_in / wt_in given)
    int nparts; long long pstride;           // logits as nparts partial sums, part p at logits + p * pstride
    const float* bias; float temp; float route_scale; int score_func; int norm;
    const int* eid_in; const float* wt_in;   // precomputed routing [M][topk] when logits is NULL
    int M, topk, E;
    int pairs;                               // M tokens through the one-token path, one workgroup row per pair
    int rows;                                // activation rows LDS holds (members staged per pass)
    const uint16_t* x; long long ldx;        // bf16 [M][H] activations on the FP8 grid
    const uint8_t* W13; long long stride_we; const uint8_t* S13; long long stride_se;
    int H, I;
    float limit;
    uint8_t* hc; long long ldhc; uint8_t* hs; long long ldhs;   // h codes [P + 1][I], E8M0 [P + 1][I / 32]
    int* eid_out; float* wt_out;                                 // routing [M][topk]
    int* grp_expert; int* grp_start; int* tok_sorted; float* wt_sorted;   // tables, P = M * topk slots
    // SH: the bf16 shared expert's gate/up GEMV rides in the same launch: grid rows 0 .. sh_y - 1 are its 16-row
    // blocks of Ws13 (2 I rows, bf16 [2I][ldws]), each over the full K; gus = bf16(x . Ws13^T) [M][ldgus]
    const uint16_t* Ws13; long long ldws; uint16_t* gus; long long ldgus; int sh_y;
    int sh_tiled;   // Ws13 in 16 x 32 tiles of 1 KiB ([2I/16][H/32][16][32], ldws = H) instead of row-major
    // SH == 2: the shared expert's [w1; w3] is FP8 E4M3 (Ws13 read as bytes, ldws = H bytes per row) in the w8 tile
    // order [2I/16][H/64][4][16][16 B], with E8M0 scales Ss13 [2I/32][ldss] per 32 x 32 block
    const uint8_t* Ss13; long long ldss;
};

// One 16-row block of the shared expert's [w1; w3] (bf16) over the full K for M tokens: the 8 waves split K into
// contiguous 32-k chunk ranges, stream 16 x 64-byte row pieces per bf16 MFMA (1 KiB per wave-load) with the token
// rows as the B operand, and sum through LDS in wave order; gate/up are stored rounded to bf16 (the shared expert's
// F.linear output is a bf16 tensor, decode.py:368, w8.py:102-103). These workgroups need no routing, so their
// weight streams start at kernel entry, while the routed workgroups still run the gate.
template <int PF>
__device__ __forceinline__ void shared_up_unit(const DecodeUpArgs& a, v4f (*s_red)[64]) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = blockIdx.y * gridDim.x + blockIdx.x;            // 16-row block of Ws13
    const int nc = a.H >> 5;                                        // 32-k chunks
    const int c0 = nc * wave / UP_WAVES, c1 = nc * (wave + 1) / UP_WAVES;
    const int col = lane & 15, kb = lane >> 4;
    // a lane's 16 bytes of chunk c: row col, k [32 c + 8 kb, +8); tiled: at 1024 c + 64 col + 16 kb of the row block
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.Ws13 + (long long)rb * 16 * a.ldws, (uint32_t)(16 * a.ldws * 2));
    const uint32_t cs = a.sh_tiled ? 1024u : 64u;
    const uint32_t wv = (uint32_t)(a.sh_tiled ? col * 64 + kb * 16 : (col * a.ldws + kb * 8) * 2) + (uint32_t)c0 * cs;
    const bool ok = col < a.M;                                      // columns past the tokens read row 0, unused
    const uint16_t* xr = a.x + (long long)(ok ? col : 0) * a.ldx + kb * 8 + (long long)c0 * 32;
    v4i A[PF], B[PF];
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    pipelined<PF>(c1 - c0,
        [&](int slot, int c) {
            A[slot] = buffer_load_tile(wr, wv, (uint32_t)c * cs);
            B[slot] = *(const v4i*)(xr + (long long)c * 32);
        },
        [&](int slot) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, A[slot]), __builtin_bit_cast(v8bf, B[slot]), acc, 0, 0, 0);
        });
    s_red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0 || !ok) return;
    v4f sum = s_red[0][lane];
#pragma unroll
    for (int w = 1; w < UP_WAVES; ++w) sum += s_red[w][lane];
    uint16_t* o = a.gus + (long long)col * a.ldgus + rb * 16 + 4 * kb;
    o[0] = (uint16_t)f32_to_bf16_bits(sum.x);
    o[1] = (uint16_t)f32_to_bf16_bits(sum.y);
    o[2] = (uint16_t)f32_to_bf16_bits(sum.z);
    o[3] = (uint16_t)f32_to_bf16_bits(sum.w);
}

// The same unit for an FP8 shared expert: 64-k chunks of 1 KiB (lane l holds row l % 16, k 16 (l / 16) .. +15), each
// decoded with its 32 x 32 block's scale into two bf16 MFMA operands (decode16: exact), against the token rows at the
// same k. Gate/up are stored rounded to bf16, as linear_w's FP8 GEMM returns them (w8.py:102-113).
template <int PF>
__device__ __forceinline__ void shared_up_unit_fp8(const DecodeUpArgs& a, v4f (*s_red)[64]) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = blockIdx.y * gridDim.x + blockIdx.x;            // 16-row block of Ws13
    const int nc = a.H >> 6;                                        // 64-k chunks
    const int c0 = nc * wave / UP_WAVES, c1 = nc * (wave + 1) / UP_WAVES;
    const int col = lane & 15, kb = lane >> 4;
    const uint8_t* W = (const uint8_t*)a.Ws13;
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(W + (long long)rb * 16 * a.ldws, (uint32_t)(16 * a.ldws));
    const uint32_t wv = (uint32_t)lane * 16u + (uint32_t)c0 * 1024u;
    const bool ok = col < a.M;                                      // columns past the tokens read row 0, unused
    const uint16_t* xr = a.x + (long long)(ok ? col : 0) * a.ldx + kb * 16 + (long long)c0 * 64;
    const uint8_t* sr = a.Ss13 + (long long)(rb >> 1) * a.ldss + 2 * c0 + (kb >> 1);
    v4i A[PF], X0[PF], X1[PF];
    int SB[PF];
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    pipelined<PF>(c1 - c0,
        [&](int slot, int c) {
            A[slot] = buffer_load_tile(wr, wv, (uint32_t)c * 1024u);
            SB[slot] = sr[2 * c];
            X0[slot] = *(const v4i*)(xr + (long long)c * 64);
            X1[slot] = *(const v4i*)(xr + (long long)c * 64 + 8);
        },
        [&](int slot) {
            v8bf16_t lo, hi;
            decode16(A[slot], e8m0_to_f32((uint32_t)SB[slot]), lo, hi);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, __builtin_bit_cast(v8bf, X0[slot]), acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, __builtin_bit_cast(v8bf, X1[slot]), acc, 0, 0, 0);
        });
    s_red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0 || !ok) return;
    v4f sum = s_red[0][lane];
#pragma unroll
    for (int w = 1; w < UP_WAVES; ++w) sum += s_red[w][lane];
    uint16_t* o = a.gus + (long long)col * a.ldgus + rb * 16 + 4 * kb;
    o[0] = (uint16_t)f32_to_bf16_bits(sum.x);
    o[1] = (uint16_t)f32_to_bf16_bits(sum.y);
    o[2] = (uint16_t)f32_to_bf16_bits(sum.z);
    o[3] = (uint16_t)f32_to_bf16_bits(sum.w);
}

template <int TILED, int PF, int PER, int EARLY, int SCL, int SH>
__global__ void __launch_bounds__(UP_WAVES * 64, 4) moe_decode_up_kernel(const DecodeUpArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];   // staged activation rows (codes) then their E8M0 bytes
    __shared__ int s_eid[UP_MAXM * UP_MAXK];
    __shared__ float s_wt[UP_MAXM * UP_MAXK];
    __shared__ unsigned long long s_bits[UP_MAXE / 64];   // selected experts
    __shared__ int s_tok[UP_MAXM * UP_MAXK], s_slot[UP_MAXM * UP_MAXK];   // members of this workgroup's group
    __shared__ float s_pw[UP_MAXM * UP_MAXK];
    __shared__ int s_pick, s_xready;
    __shared__ unsigned long long s_wmem[UP_WAVES], s_wlow[UP_WAVES];   // per wave: member / smaller-expert pair ballots
    __shared__ v4f s_acc[UP_WAVES][64];
    __shared__ __align__(16) uint8_t s_wsc[SCL ? UP_WAVES * UP_WSC : 16];
    if (SH && (int)blockIdx.y < a.sh_y) {   // a shared-expert row block (uniform over the workgroup)
        if (SH == 2) shared_up_unit_fp8<6>(a, s_acc);
        else shared_up_unit<8>(a, s_acc);
        return;
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform values kept in scalar registers
    const int M = a.M, topk = a.topk, P = M * a.topk, E = a.E;
    const int K = a.H, nk = K >> 7, Kh = K >> 1, Ks = K >> 5, LS = K + 16;
    uint8_t* lds_s = smem + a.rows * LS;

    // Activation row `row` of LDS <- token `tok`: E4M3 codes + E8M0 bytes. Two lanes per 32-value group,
    // 16 values (2 x 16 bytes) each; a lane pair is always active together. load / convert are split so the
    // loads can be issued early.
    const int per_row = Ks * 2;
    auto x_load = [&](int tok, int q, v4i& r0, v4i& r1) {
        const uint16_t* src = a.x + (long long)tok * a.ldx + q * 16;
        r0 = *(const v4i*)src;
        r1 = *(const v4i*)(src + 8);
    };
    auto x_store = [&](int row, int q, v4i r0, v4i r1) {
        const uint32_t wd[8] = {(uint32_t)r0.x, (uint32_t)r0.y, (uint32_t)r0.z, (uint32_t)r0.w,
                                (uint32_t)r1.x, (uint32_t)r1.y, (uint32_t)r1.z, (uint32_t)r1.w};
        float f[16];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            f[2 * j] = bf16_to_f32(wd[j] & 0xFFFFu);
            f[2 * j + 1] = bf16_to_f32(wd[j] >> 16);
        }
        float amax = 0.f;
#pragma unroll
        for (int j = 0; j < 16; ++j) amax = fmaxf(amax, fabsf(f[j]));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 2));
        const int e = fq8_exponent(amax);
        uint32_t cw[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) cw[j] = fq8_code4_hw(f[4 * j], f[4 * j + 1], f[4 * j + 2], f[4 * j + 3], e);
        *(v4i*)(smem + row * LS + q * 16) = v4i{(int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3]};
        if ((q & 1) == 0) lds_s[row * Ks + (q >> 1)] = (uint8_t)(e + 127);
    };

    // ---- one token (EARLY): wave gw runs the gate while the other seven waves stage the token's activations in LDS
    // row 0. The gate is the critical path, so wave gw issues the logits loads first, before the barrier below.
    // `early` is compile-time, so the one-token instantiation holds none of the member-pass code (the host launches
    // EARLY only for M == 1 and per_row <= (UP_WAVES - 1) * 64).
    constexpr bool early = EARLY != 0;
    GateRow<PER> gr;
    // the wave that runs the gate rotates with the workgroup index (waves 0-3 sit on different SIMDs), so the two
    // workgroups a CU holds do not run their gates on the same SIMD
    const int gw = (int)((blockIdx.x + blockIdx.y * gridDim.x) & 3);
    const int g = (int)blockIdx.y - (SH ? a.sh_y : 0);   // this workgroup's group slot (the g-th selected expert)
    // The one-token path also serves M tokens pair by pair (a.pairs): row g is then pair g = pick pk of token tok, whose
    // h row is g itself (no bucketing: an expert two tokens share streams once per pair). One token: tok 0, pick g.
    const int tok = early ? g / topk : 0, pk = early ? g - tok * topk : g;
    const float* lrow = a.logits ? a.logits + (long long)tok * a.ldl : nullptr;
    const bool gwave = early && wave == gw;
    if (gwave && a.logits) gr.load_logits(lrow, E, a.nparts, a.pstride);
    const int xq = (wave - (wave > gw ? 1 : 0)) * 64 + lane;   // early: the lane's 16 values of row 0 among the stagers
    v4i xr0, xr1;
    if (early && !gwave && xq < per_row) x_load(tok, xq, xr0, xr1);
    if (tid < UP_MAXE / 64) s_bits[tid] = 0ull;
    if (tid == 0) {
        s_pick = -2;
        s_xready = 0;
    }
    if (early) __syncthreads();   // s_pick, s_xready and s_bits are set before any wave uses them

    // ---- this wave's weight stream: row block rb of {gate c0, gate c0 + 16, up c0, up c0 + 16}, K-half kh; the
    // expert (the buffer descriptors) comes from the routing
    const int c0 = blockIdx.x * 32;
    const int rbi = wave & 3, kh = wave >> 2;
    const int row_first = (rbi < 2 ? c0 : a.I + c0) + (rbi & 1) * 16;
    const int nb = row_first >> 4;
    const int nk_h = nk / 2, k0c = kh * nk_h, nk_w = kh ? nk - nk_h : nk_h;
    const uint32_t wv = (uint32_t)wtile_off<TILED>(nb, k0c, nk, Kh, lane), sv = (uint32_t)stile_off<TILED>(nb, k0c, nk, Ks, lane);
    const int ws = TILED ? 1024 : 64, ss = TILED ? 64 : 4;
    const int col = lane & 15, kb = lane >> 4;
    __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.W13, 0u), sr = buffer_rsrc(a.S13, 0u);
    auto set_expert = [&](int e) {
        wr = buffer_rsrc(a.W13 + (long long)e * a.stride_we, (uint32_t)a.stride_we);
        sr = buffer_rsrc(a.S13 + (long long)e * a.stride_se, (uint32_t)a.stride_se);
    };
    v4i A[PF];
    int SA[PF];
    auto load = [&](int slot, int kc) {
        A[slot] = buffer_load_tile(wr, wv, (uint32_t)(kc * ws));
        if (!SCL) SA[slot] = buffer_load_byte(sr, sv, (uint32_t)(kc * ss));
    };
    // SCL (always for one token; for M tokens when a wave's stream has <= 32 k-chunks): a wave's E8M0 bytes (16
    // rows x nk_w k-chunks) are fetched with a few wide loads when its expert is known, ahead of its first tiles,
    // and kept in LDS in MFMA order (k-chunk j at 64 j, row r's byte for k-block kb at 4 r + kb), so each k-step
    // reads its scale from LDS instead of issuing a byte load per lane: the byte loads cost as much load-unit
    // time as the weight tiles themselves.
    uint8_t* const wsc = s_wsc + (SCL ? wave * UP_WSC : 0);
    v4i SC[TILED ? 2 : 8];
    auto scale_load = [&]() {
        if (TILED) {   // the stream's bytes are contiguous: (nb nk + k0c) 64 .. + 64 nk_w
            // lanes past the stream's nk_w * 64 bytes get an offset past the descriptor: no fetch, zeros
            const uint32_t b = (uint32_t)stile_off<1>(nb, k0c, nk, Ks, 0) + lane * 16;
            SC[0] = buffer_load_tile(sr, lane * 16 < nk_w * 64 ? b : 0xFFFFFFF0u, 0);
            SC[1] = buffer_load_tile(sr, 1024 + lane * 16 < nk_w * 64 ? b + 1024 : 0xFFFFFFF0u, 0);
        } else {       // row r's bytes k0c 4 .. are contiguous: one dword (4 k-blocks) per (row, k-chunk)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int idx = 64 * i + lane, r = idx & 15, j = idx >> 4;
                SC[i].x = (int)__builtin_amdgcn_raw_buffer_load_b32(sr, j < nk_w ? (uint32_t)((nb * 16 + r) * Ks + (k0c + j) * 4) : 0xFFFFFFF0u, 0, 0);
            }
        }
    };
    auto scale_store = [&]() {
        if (TILED) {
            *(v4i*)(wsc + lane * 16) = SC[0];
            *(v4i*)(wsc + 1024 + lane * 16) = SC[1];
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int idx = 64 * i + lane, r = idx & 15, j = idx >> 4;
                *(int*)(wsc + j * 64 + r * 4) = SC[i].x;
            }
        }
    };

    // ---- routing, identical in every workgroup.
    // One token (early): wave gw runs the gate; this workgroup's expert is the g-th pick, which wave gw posts in LDS
    // right after round g, so every wave's weight tiles go out while the later rounds run. (Its h row is still
    // the expert's rank in ascending id order, which wave gw finds once all rounds are done.)
    // M tokens: one wave per token; the workgroup's expert is the g-th smallest selected id.
    int eg = -1;
    if (early) {
        if (gwave) {
            int ki = -1;
            float kw = 0.f;   // lane k keeps pick k
            if (a.logits) {
                gr.prepare(lrow, a.nparts, a.pstride, a.bias, E, a.temp, a.score_func);
                float wsum = 0.f;
                for (int k = 0; k < topk; ++k) {
                    int id;
                    float w;
                    gr.pick(k, &id, &w);
                    wsum += w;
                    if (k == pk) {
                        eg = (id >= 0 && id < E) ? id : -1;
                        if (lane == 0) __hip_atomic_store(&s_pick, eg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                        if (eg >= 0) {
                            set_expert(eg);
                            scale_load();
                            pipeline_start<PF>(nk_w, load);
                        }
                    }
                    if (lane == k) { ki = id; kw = w; }
                }
                kw = gate_weight(kw, wsum, a.route_scale, a.norm);
            } else {
                if (lane < topk) {
                    ki = a.eid_in[tok * topk + lane];
                    kw = a.wt_in[tok * topk + lane];
                }
                eg = __builtin_amdgcn_readfirstlane(a.eid_in[g]);
                if (!(eg >= 0 && eg < E)) eg = -1;
                if (eg >= 0) {
                    set_expert(eg);
                    scale_load();
                    pipeline_start<PF>(nk_w, load);
                }
            }
            // the routing of the token, the selected-expert mask, and this workgroup's member: its h row is the
            // expert's rank among the selected ids (ascending), its weight that of the first pair holding the expert
            const bool kv = lane < topk && ki >= 0 && ki < E;   // out-of-range ids are dropped, never read
            if (lane < topk) {
                s_eid[lane] = kv ? ki : -1;
                s_wt[lane] = kw;
            }
            if (kv) atomicOr(&s_bits[ki >> 6], 1ull << (ki & 63));
            const int rank = __popcll(__ballot(kv && ki < eg));
            const unsigned long long mine = __ballot(kv && ki == eg);
            const float pw = __shfl(kw, a.pairs ? pk : (mine ? (int)__builtin_ctzll(mine) : 0));
            if (lane == 0) {
                s_slot[0] = a.pairs ? g : rank;
                s_pw[0] = pw;
            }
            if (eg >= 0) scale_store();   // its scale loads went out with the first tiles, at the pick
        } else {
            // stage this wave's part of row 0 (the loads went out at kernel start), release it, then follow the pick
            if (xq < per_row) x_store(0, xq, xr0, xr1);
            if (lane == 0) __hip_atomic_fetch_add(&s_xready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (a.logits) {
                // the pick, posted by wave gw (s_pick starts at -2, before the first barrier)
                while ((eg = __hip_atomic_load(&s_pick, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == -2) __builtin_amdgcn_s_sleep(1);
                eg = __builtin_amdgcn_readfirstlane(eg);
            } else {
                eg = __builtin_amdgcn_readfirstlane(a.eid_in[g]);
                if (!(eg >= 0 && eg < E)) eg = -1;
            }
            if (eg >= 0) {
                set_expert(eg);
                // the first PF tiles, issued as pipeline_start does but without its short-stream branch, so the store
                // below sits in the same block and waits for the two scale loads only (older than every tile). With
                // fewer than PF k-chunks (small K) the extra loads read other bytes of the expert or zeros past its
                // end, and pipeline_finish's unpipelined path loads what it uses again.
                scale_load();
#pragma unroll
                for (int i = 0; i < PF; ++i) {
                    load(i, i);
                    __builtin_amdgcn_sched_barrier(0);
                }
                scale_store();
            }
        }
    } else {
        for (int t = wave; t < M; t += UP_WAVES) {
            int ki = 0;
            float kw = 0.f;
            if (a.logits) {
                gate_row_wave<PER>(a.logits + (long long)t * a.ldl, a.nparts, a.pstride, a.bias, E, a.temp, topk, a.route_scale, a.score_func,
                                   a.norm, &ki, &kw);
            } else if (lane < topk) {
                ki = a.eid_in[t * topk + lane];
                kw = a.wt_in[t * topk + lane];
            }
            if (lane < topk) {
                s_eid[t * topk + lane] = (ki >= 0 && ki < E) ? ki : -1;   // out-of-range ids are dropped, never read
                s_wt[t * topk + lane] = kw;
            }
        }
    }
    // the tables of the down projection: one token, workgroup (0, 0) writes them all; pairs, workgroup (0, g) the entries
    // of pair g (group g = that pair alone)
    const bool publish = blockIdx.x == 0 && (g == 0 || a.pairs);
    int mg = 1;
    if (early) {
        if (eg < 0 && !publish) return;   // uniform: an invalid id (given routing only)
    } else {
        __syncthreads();
        for (int p = tid; p < P; p += blockDim.x) {
            const int e = s_eid[p];
            if (e >= 0) atomicOr(&s_bits[e >> 6], 1ull << (e & 63));
        }
        __syncthreads();

        // ---- the selected experts (groups are in ascending expert order); this workgroup's is the g-th
        int U = 0;
#pragma unroll
        for (int w = 0; w < UP_MAXE / 64; ++w) {
            unsigned long long bits = s_bits[w];
            bits = ((unsigned long long)(unsigned)__builtin_amdgcn_readfirstlane((int)(bits >> 32)) << 32) |
                   (unsigned)__builtin_amdgcn_readfirstlane((int)(unsigned)bits);
            const int c = __popcll(bits);
            if (eg < 0 && g < U + c) {
                for (int r = g - U; r > 0; --r) bits &= bits - 1ull;   // drop the lower set bits
                eg = 64 * w + (int)__builtin_ctzll(bits);
            }
            U += c;
        }
        if (g >= U && !publish) return;   // uniform: fewer experts than slots
        if (g < U) {
            set_expert(eg);
            if (SCL) scale_load();   // lands while the members are found and their rows staged
        }

        // ---- members of the group (tokens holding expert eg, ascending) and their sorted pair slots. Thread p looks at
        // pair p (P <= 256 of 512 threads): ballots give the pairs of a smaller expert (the group's first slot) and
        // the members before p (its rank; pairs are token-major, so in token order), in one pass
        const int ep = (g < U && tid < P) ? s_eid[tid] : -1;
        const bool is_mem = ep >= 0 && ep == eg;
        const unsigned long long bmem = __ballot(is_mem), blow = __ballot(ep >= 0 && ep < eg);
        if (lane == 0) {
            s_wmem[wave] = bmem;
            s_wlow[wave] = blow;
        }
        __syncthreads();
        int lt = 0, before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < UP_WAVES; ++w) {
            const int c = __popcll(s_wmem[w]);
            lt += __popcll(s_wlow[w]);
            before += w < wave ? c : 0;
            total += c;
        }
        if (is_mem) {
            const int same = before + __popcll(bmem & ((1ull << lane) - 1ull));
            s_tok[same] = tid / topk;
            s_slot[same] = lt + same;
            s_pw[same] = s_wt[tid];
        }
        __syncthreads();
        mg = g < U ? __builtin_amdgcn_readfirstlane(total) : 0;
    }
    const bool work = eg >= 0;

    const uint8_t* xl;
    const uint8_t* xsl;
    const uint8_t* wsl;   // SCL: this lane's weight scale of the next k-chunk
    v4f acc;
    auto use = [&](int slot) {
        const v4i b0 = *(const v4i*)(xl);
        const v4i b1 = *(const v4i*)(xl + 64);
        const int sb = *xsl;
        const int sa = SCL ? (int)*wsl : SA[slot];
        xl += 128;
        xsl += 4;
        if (SCL) wsl += 64;
        acc = mfma_fp4w_fp8x(v8i{A[slot].x, A[slot].y, A[slot].z, A[slot].w, 0, 0, 0, 0},
                             v8i{b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w}, acc, sa, sb);
    };
    // B column c = member base + c of the pass (columns past the pass read row 0; their results are unused)
    auto start_pass = [&](int mp) {
        const int brow = col < mp ? col : 0;
        xl = smem + brow * LS + k0c * 128 + kb * 16;
        xsl = lds_s + brow * Ks + k0c * 4 + kb;
        wsl = wsc + (lane & 15) * 4 + kb;
        acc = v4f{0.f, 0.f, 0.f, 0.f};
    };
    // SwiGLU epilogue: half-wave i handles member base + i; lane c of it handles column c0 + c
    auto epilogue = [&](int base, int mp) {
        s_acc[wave][lane] = acc;
        __syncthreads();
        const int hw = tid >> 5, c = tid & 31;
        if (hw < mp) {
            // D[row][col] of a 16x16 accumulator sits in lane col + 16 (row / 4), element row % 4
            const int r16 = c & 15, l = hw + 16 * (r16 >> 2), el = r16 & 3;
            const int wg = c >> 4;   // gate row block of column c (0 / 1), up block = 2 + wg
            float gg = s_acc[wg][l][el] + s_acc[4 + wg][l][el];
            float uu = s_acc[2 + wg][l][el] + s_acc[6 + wg][l][el];
            if (a.limit > 0.f) {
                uu = fminf(fmaxf(uu, -a.limit), a.limit);
                gg = fminf(gg, a.limit);
            }
            float h = gg * (1.0f / (1.0f + expf(-gg))) * uu;
            h = h * s_pw[base + hw];
            h = bf16_round(h);
            const int e = fq8_exponent(wave_max32(fabsf(h)));
            const int slot = s_slot[base + hw];
            a.hc[(long long)slot * a.ldhc + c0 + c] = (uint8_t)fq8_code(h, e);
            if (c == 0) a.hs[(long long)slot * a.ldhs + (c0 >> 5)] = (uint8_t)(e + 127);
        }
    };

    if (early) {
        // one token: the first tiles are in flight; the stream starts once the seven stagers have released row 0,
        // without waiting for the rest of the top-k (the gate wave joins when its rounds are done). A token's
        // expert ids are distinct, as the gate guarantees, so the group has one member, whose h row and weight the
        // gate wave has written before it reaches the epilogue's barrier.
        if (work) {
            while (__hip_atomic_load(&s_xready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < UP_WAVES - 1) __builtin_amdgcn_s_sleep(1);
            start_pass(1);
            pipeline_finish<PF>(nk_w, load, use);
            epilogue(0, 1);
        } else {
            __syncthreads();   // (publishing workgroup only) the gate wave's routing and mask are visible
        }
    } else {
        // passes of up to a.rows members (16 B columns); a group with more members than LDS rows holds (possible
        // only when many tokens share an expert) streams the expert's weights once per pass
        auto stage = [&](int base, int mp) {
#pragma unroll 1
            for (int i = tid; i < mp * per_row; i += blockDim.x) {
                const int r = i / per_row, q = i - r * per_row;
                v4i r0, r1;
                x_load(s_tok[base + r], q, r0, r1);
                x_store(r, q, r0, r1);
            }
            if (SCL && base == 0) scale_store();   // its loads are older than the rows just staged
            __syncthreads();
        };
        // (M tokens keep 4 tiles in flight per wave: in-process A/B at M = 4 / 16, 8 tiles in the one-pass case
        // ran 1.7 % / 2.5 % slower)
        if (work && mg <= a.rows) {   // one pass (the common case), outside the pass loop
            stage(0, mg);
            start_pass(mg);
            pipelined<PF>(nk_w, load, use);
            epilogue(0, mg);
        } else if (work) {
            for (int base = 0; base < mg; base += a.rows) {
                const int mp = min(a.rows, mg - base);
                if (base > 0) __syncthreads();   // LDS rows are reused
                stage(base, mp);
                start_pass(mp);
                pipelined<PF>(nk_w, load, use);
                epilogue(base, mp);
            }
        }
    }

    // ---- pairs: pair g's routing and table entries (group g holds pair g alone; an invalid id makes it an empty group)
    if (publish && a.pairs) {
        if (tid == 0) {
            const int e = s_eid[pk];
            const float w = s_wt[pk];
            if (a.eid_out) a.eid_out[g] = e;
            if (a.wt_out) a.wt_out[g] = w;
            a.grp_expert[g] = e;
            a.grp_start[g] = g;
            a.tok_sorted[g] = tok;
            a.wt_sorted[g] = w;
            if (g == 0) a.grp_start[P] = P;
        }
        return;
    }
    // ---- workgroup (0, 0) publishes the routing and the tables of the down projection (off the critical path:
    // the down projection is the next launch)
    if (publish) {
        int U = 0;   // selected experts
#pragma unroll
        for (int w = 0; w < UP_MAXE / 64; ++w) U += __popcll(s_bits[w]);
        int valid = 0;
        for (int p = 0; p < P; ++p) valid += s_eid[p] >= 0 ? 1 : 0;
        for (int p = tid; p < P; p += blockDim.x) {
            const int e = s_eid[p];
            if (a.eid_out) a.eid_out[p] = e;
            if (a.wt_out) a.wt_out[p] = s_wt[p];
            if (e < 0) continue;
            int lt = 0, same = 0;
            for (int q = 0; q < P; ++q) {
                const int eq = s_eid[q];
                lt += (eq >= 0 && eq < e) ? 1 : 0;
                same += (eq == e && q < p) ? 1 : 0;
            }
            a.tok_sorted[lt + same] = p / topk;
            a.wt_sorted[lt + same] = s_wt[p];
            if (same == 0) {   // first pair of its expert: the group entry; group index = selected ids below e
                int gi = 0;
                for (int w = 0; w < (e >> 6); ++w) gi += __popcll(s_bits[w]);
                gi += __popcll(s_bits[e >> 6] & ((1ull << (e & 63)) - 1ull));
                a.grp_expert[gi] = e;
                a.grp_start[gi] = lt;
            }
        }
        for (int s2 = U + tid; s2 < P; s2 += blockDim.x) { a.grp_expert[s2] = -1; a.grp_start[s2] = valid; }
        if (tid == 0) { a.grp_start[U] = valid; a.grp_start[P] = valid; }
        for (int s2 = valid + tid; s2 < P; s2 += blockDim.x) { a.tok_sorted[s2] = 0; a.wt_sorted[s2] = 0.f; }
    }
}

static int decode_up_launch(const float* logits, long long ldl, int nparts, long long part_stride, const float* bias, float temp,
                            float route_scale, int score_func, int norm, const int* eid_in, const float* wt_in, int M, int topk, int E, const uint16_t* x,
                            long long ldx, const uint8_t* W13, long long stride_we, const uint8_t* S13, long long stride_se,
                            int tiled, int H, int I, float limit, uint8_t* hc, long long ldhc, uint8_t* hs, long long ldhs,
                            int* eid_out, float* wt_out, int* grp_expert, int* grp_start, int* tok_sorted, float* wt_sorted,
                            const uint16_t* Ws13, long long ldws, int sh_tiled, uint16_t* gus, long long ldgus, const uint8_t* Ss13,
                            long long ldss13, bool pairs, void* stream) {
    if ((!logits && (!eid_in || !wt_in)) || !x || !W13 || !S13 || !hc || !hs || !grp_expert || !grp_start || !tok_sorted || !wt_sorted)
        return DSV41_EINVAL;
    if (M < 1 || M > UP_MAXM || topk < 1 || topk > UP_MAXK || topk > E || E < 1 || E > UP_MAXE || score_func < 0 || score_func > 2)
        return DSV41_EINVAL;
    if (logits && (nparts < 1 || (nparts > 1 && part_stride < (long long)M * ldl))) return DSV41_EINVAL;
    if (H <= 0 || (H & 255) || I <= 0 || (I & 31) || ldx < H || (ldx & 7) || (((uintptr_t)x) & 15) || (logits && ldl < E)) return DSV41_EINVAL;
    // every h row holds I codes and I / 32 scale bytes (the epilogue writes columns 0 .. I - 1 of each)
    if (ldhc < I || ldhs < I / 32) return DSV41_EINVAL;
    // the shared expert's [w1; w3] (bf16 [2I][ldws]) and its gate/up output (bf16 [M][ldgus]): 16-row blocks addressed
    // with 32-bit offsets, 16-byte row pieces
    const bool sh_fp8 = Ws13 && Ss13;
    if (Ws13 && !sh_fp8 && (!gus || ldws < H || (ldws & 7) || (((uintptr_t)Ws13) & 15) || 16 * ldws * 2 > 0xFFFFFFFFll || ldgus < 2 * I ||
                            (sh_tiled && ldws != H)))
        return DSV41_EINVAL;
    // FP8 shared expert: E4M3 bytes in the w8 tile order (ldws = H bytes per row), E8M0 [2I/32][ldss13]
    if (sh_fp8 && (!gus || !sh_tiled || ldws != H || (((uintptr_t)Ws13) & 15) || 16LL * ldws > 0xFFFFFFFFll || ldgus < 2 * I ||
                   ldss13 < H / 32 || (I & 15)))
        return DSV41_EINVAL;
    // one expert's weights must be addressable with 32-bit offsets, and hold 2 I rows of H / 2 bytes
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll ||
        stride_we < (long long)2 * I * (H / 2) || stride_se < (long long)2 * I * (H / 32)) return DSV41_EINVAL;
    // M = 1: the single token's codes are staged while the routing runs (one LDS row, H / 16 <= 448 lanes: the
    // seven waves besides the gate's).
    // M > 1: members are staged after the bucketing, up to `rows` per pass, as many as fit in 44 KiB of LDS (60 KiB
    // without the staged weight scales), so two workgroups fit per CU
    const size_t row_bytes = (size_t)(H + 16) + (size_t)(H / 32);
    // pairs: M tokens through the same path, one grid row per (token, pick) pair
    if (pairs && H / 16 > (UP_WAVES - 1) * 64) return DSV41_EINVAL;
    pairs = pairs && M > 1;
    const bool early = (M == 1 || pairs) && H / 16 <= (UP_WAVES - 1) * 64;
    // M tokens: weight scales through LDS (16 KiB per workgroup) when a wave's stream has <= 32 k-chunks; the rows
    // then get 44 KiB, so two workgroups still fit per CU
    const bool scl = early || (H / 128 + 1) / 2 <= UP_WSC / 64;
    int rows = early ? 1 : (int)(((scl ? 44 : 60) * 1024) / row_bytes);
    rows = rows > 16 ? 16 : (rows > M ? M : rows);
    if (rows < 1) return DSV41_EINVAL;
    // the shared expert's 2 I / 16 row blocks take sh_y = 4 extra grid rows of I / 32 workgroups, ahead of the routed
    // ones (the hardware dispatches workgroups in linear order, so their streams start first)
    const int sh_y = Ws13 ? (2 * I / 16) / (I / 32) : 0;
    DecodeUpArgs a{logits, ldl, nparts, part_stride, bias, temp, route_scale, score_func, norm, eid_in, wt_in, M, topk, E, pairs ? 1 : 0, rows, x, ldx, W13, stride_we, S13,
                   stride_se, H, I, limit, hc, ldhc, hs, ldhs, eid_out, wt_out, grp_expert, grp_start, tok_sorted, wt_sorted,
                   Ws13, ldws, gus, ldgus, sh_y, sh_tiled, Ss13, ldss13};
    const size_t lds = rows * row_bytes;
    const dim3 grid(I / 32, M * topk + sh_y), block(UP_WAVES * 64);
    hipStream_t st = (hipStream_t)stream;
#define UP_LAUNCH_SH(T, PER, SHV)                                                                                 \
    do {                                                                                                      \
        if (early) moe_decode_up_kernel<T, 8, PER, 1, 1, SHV><<<grid, block, lds, st>>>(a);                   \
        else if (scl) moe_decode_up_kernel<T, 4, PER, 0, 1, SHV><<<grid, block, lds, st>>>(a);                \
        else moe_decode_up_kernel<T, 4, PER, 0, 0, SHV><<<grid, block, lds, st>>>(a);                         \
    } while (0)
#define UP_LAUNCH(T, PER)                                                                                         \
    do {                                                                                                      \
        if (sh_fp8) UP_LAUNCH_SH(T, PER, 2); else if (sh_y) UP_LAUNCH_SH(T, PER, 1); else UP_LAUNCH_SH(T, PER, 0); \
    } while (0)
    if (E <= 256) { if (tiled) UP_LAUNCH(1, 4); else UP_LAUNCH(0, 4); }
    else if (E <= 384) { if (tiled) UP_LAUNCH(1, 6); else UP_LAUNCH(0, 6); }
    else { if (tiled) UP_LAUNCH(1, 8); else UP_LAUNCH(0, 8); }
#undef UP_LAUNCH
#undef UP_LAUNCH_SH
    return (int)hipGetLastError();
}

extern "C" int dsv41_moe_decode_up(const float* logits, long long ldl, int nparts, long long part_stride, const float* bias, float temp,
                                   float route_scale, int score_func, int norm, const int* eid_in, const float* wt_in, int M, int topk, int E, const uint16_t* x,
                                   long long ldx, const uint8_t* W13, long long stride_we, const uint8_t* S13, long long stride_se,
                                   int tiled, int H, int I, float limit, uint8_t* hc, long long ldhc, uint8_t* hs, long long ldhs,
                                   int* eid_out, float* wt_out, int* grp_expert, int* grp_start, int* tok_sorted, float* wt_sorted,
                                   const uint16_t* Ws13, long long ldws, int sh_tiled, uint16_t* gus, long long ldgus, const uint8_t* Ss13,
                                   long long ldss13, void* stream) {
    return decode_up_launch(logits, ldl, nparts, part_stride, bias, temp, route_scale, score_func, norm, eid_in, wt_in, M, topk, E, x, ldx, W13,
                            stride_we, S13, stride_se, tiled, H, I, limit, hc, ldhc, hs, ldhs, eid_out, wt_out, grp_expert, grp_start,
                            tok_sorted, wt_sorted, Ws13, ldws, sh_tiled, gus, ldgus, Ss13, ldss13, false, stream);
}

extern "C" int dsv41_moe_decode_up_pairs(const float* logits, long long ldl, int nparts, long long part_stride, const float* bias, float temp,
                                         float route_scale, int score_func, int norm, const int* eid_in, const float* wt_in, int M, int topk, int E,
                                         const uint16_t* x, long long ldx, const uint8_t* W13, long long stride_we, const uint8_t* S13,
                                         long long stride_se, int tiled, int H, int I, float limit, uint8_t* hc, long long ldhc, uint8_t* hs,
                                         long long ldhs, int* eid_out, float* wt_out, int* grp_expert, int* grp_start, int* tok_sorted,
                                         float* wt_sorted, const uint16_t* Ws13, long long ldws, int sh_tiled, uint16_t* gus, long long ldgus,
                                         const uint8_t* Ss13, long long ldss13, void* stream) {
    return decode_up_launch(logits, ldl, nparts, part_stride, bias, temp, route_scale, score_func, norm, eid_in, wt_in, M, topk, E, x, ldx, W13,
                            stride_we, S13, stride_se, tiled, H, I, limit, hc, ldhc, hs, ldhs, eid_out, wt_out, grp_expert, grp_start,
                            tok_sorted, wt_sorted, Ws13, ldws, sh_tiled, gus, ldgus, Ss13, ldss13, true, stream);
}
