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

#define UP_WAVES 8
#define UP_MAXM 16
#define UP_MAXK 16
#define UP_MAXE 512
#define UP_MAX_LDS (136 * 1024)   // dynamic LDS bound (gfx950: 160 KiB per workgroup, less the static arrays)

struct DecodeUpArgs {
    const float* logits; long long ldl;      // fp32 [M][E] router logits (or NULL: eid_in / wt_in given)
    const float* bias; float temp; float route_scale; int score_func; int norm;
    const int* eid_in; const float* wt_in;   // precomputed routing [M][topk] when logits is NULL
    int M, topk, E;
    int rows;                                // activation rows LDS holds (= M)
    const uint16_t* x; long long ldx;        // bf16 [M][H] activations on the FP8 grid
    const uint8_t* W13; long long stride_we; const uint8_t* S13; long long stride_se;
    int H, I;
    float limit;
    uint8_t* hc; long long ldhc; uint8_t* hs; long long ldhs;   // h codes [P + 1][I], E8M0 [P + 1][I / 32]
    int* eid_out; float* wt_out;                                 // routing [M][topk]
    int* grp_expert; int* grp_start; int* tok_sorted; float* wt_sorted;   // tables, P = M * topk slots
};

template <int TILED, int PF, int PER>
__global__ void __launch_bounds__(UP_WAVES * 64, 4) moe_decode_up_kernel(const DecodeUpArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];   // staged activation rows (codes) then their E8M0 bytes
    __shared__ int s_eid[UP_MAXM * UP_MAXK];
    __shared__ float s_wt[UP_MAXM * UP_MAXK];
    __shared__ int s_pos[UP_MAXM * UP_MAXK];          // sorted slot of pair p
    __shared__ int s_lt[UP_MAXM * UP_MAXK];           // pairs with a smaller expert id (= group start)
    __shared__ int s_gidx[UP_MAXE];                   // group index of a selected expert
    __shared__ int s_wsum[UP_WAVES];
    __shared__ int s_tok[UP_MAXM * UP_MAXK], s_slot[UP_MAXM * UP_MAXK];   // members of this workgroup's group
    __shared__ float s_pw[UP_MAXM * UP_MAXK];
    __shared__ int s_eg, s_mg, s_ng;
    __shared__ v4f s_acc[UP_WAVES][64];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform values kept in scalar registers
    const int M = a.M, topk = a.topk, P = M * a.topk, E = a.E;

    // ---- routing for all M tokens (one wave per token), identical in every workgroup
    for (int t = wave; t < M; t += UP_WAVES) {
        int ki = 0;
        float kw = 0.f;
        if (a.logits) {
            gate_row_wave<PER>(a.logits + (long long)t * a.ldl, a.bias, E, a.temp, topk, a.route_scale, a.score_func, a.norm, &ki, &kw);
        } else if (lane < topk) {
            ki = a.eid_in[t * topk + lane];
            kw = a.wt_in[t * topk + lane];
        }
        if (lane < topk) {
            s_eid[t * topk + lane] = (ki >= 0 && ki < E) ? ki : -1;   // out-of-range ids are dropped, never read
            s_wt[t * topk + lane] = kw;
        }
    }
    for (int e = tid; e < E; e += blockDim.x) s_gidx[e] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += blockDim.x)
        if (s_eid[p] >= 0) s_gidx[s_eid[p]] = 1;
    __syncthreads();
    // ---- bucketing: group index of each selected expert (ballot prefix over experts, ascending ids)
    {
        int base = 0;
        for (int e0 = 0; e0 < E; e0 += blockDim.x) {
            const int e = e0 + tid;
            const int mark = e < E ? s_gidx[e] : 0;
            const unsigned long long bal = __ballot(mark);
            if (lane == 0) s_wsum[wave] = __popcll(bal);
            __syncthreads();
            int before = base;
            for (int w = 0; w < wave; ++w) before += s_wsum[w];
            int total = 0;
            for (int w = 0; w < UP_WAVES; ++w) total += s_wsum[w];
            const unsigned long long below = lane == 63 ? ~0ull >> 1 : ((1ull << lane) - 1ull);
            if (e < E) s_gidx[e] = mark ? before + __popcll(bal & below) : -1;
            base += total;
            __syncthreads();
        }
        if (tid == 0) s_ng = base;
    }
    // sorted slot of every pair: pairs of smaller experts first, then same expert with a smaller token
    for (int p = tid; p < P; p += blockDim.x) {
        const int e = s_eid[p];
        int lt = 0, same = 0;
        for (int q = 0; q < P; ++q) {
            const int eq = s_eid[q];
            lt += (eq >= 0 && eq < e) ? 1 : 0;
            same += (eq == e && q < p) ? 1 : 0;   // pairs are token-major: q < p = earlier token (or slot)
        }
        s_lt[p] = lt;
        s_pos[p] = e >= 0 ? lt + same : -1;
    }
    __syncthreads();
    const int U = __builtin_amdgcn_readfirstlane(s_ng);
    const int g = blockIdx.y;
    // ---- workgroup (0, 0) publishes the routing and the tables of the down projection
    if (blockIdx.x == 0 && g == 0) {
        int valid = 0;
        for (int p = 0; p < P; ++p) valid += s_eid[p] >= 0 ? 1 : 0;
        for (int p = tid; p < P; p += blockDim.x) {
            if (a.eid_out) a.eid_out[p] = s_eid[p];
            if (a.wt_out) a.wt_out[p] = s_wt[p];
            if (s_pos[p] >= 0) {
                a.tok_sorted[s_pos[p]] = p / topk;
                a.wt_sorted[s_pos[p]] = s_wt[p];
                if (s_pos[p] == s_lt[p]) {   // first pair of its expert: the group entry
                    a.grp_expert[s_gidx[s_eid[p]]] = s_eid[p];
                    a.grp_start[s_gidx[s_eid[p]]] = s_lt[p];
                }
            }
        }
        for (int s2 = U + tid; s2 < P; s2 += blockDim.x) { a.grp_expert[s2] = -1; a.grp_start[s2] = valid; }
        if (tid == 0) { a.grp_start[U] = valid; a.grp_start[P] = valid; }
        for (int s2 = valid + tid; s2 < P; s2 += blockDim.x) { a.tok_sorted[s2] = 0; a.wt_sorted[s2] = 0.f; }
    }
    if (g >= U) return;   // uniform: fewer distinct experts than slots
    // ---- this group's expert and tokens (ascending)
    if (tid < E && s_gidx[tid] == g) s_eg = tid;
    for (int e = tid + blockDim.x; e < E; e += blockDim.x)
        if (s_gidx[e] == g) s_eg = e;
    __syncthreads();
    const int eg = __builtin_amdgcn_readfirstlane(s_eg);
    if (tid == 0) s_mg = 0;
    __syncthreads();
    for (int p = tid; p < P; p += blockDim.x)
        if (s_eid[p] == eg) {   // member rank = sorted slot - group start (token order)
            const int r = s_pos[p] - s_lt[p];
            s_tok[r] = p / topk;
            s_slot[r] = s_pos[p];
            s_pw[r] = s_wt[p];
            atomicAdd(&s_mg, 1);
        }
    __syncthreads();
    const int mg = __builtin_amdgcn_readfirstlane(s_mg);

    // ---- this wave's weight stream: row block rb of {gate c0, gate c0 + 16, up c0, up c0 + 16}, K-half kh
    const int K = a.H, nk = K >> 7, Kh = K >> 1, Ks = K >> 5, LS = K + 16;
    const int c0 = blockIdx.x * 32;
    const int rbi = wave & 3, kh = wave >> 2;
    const int row_first = (rbi < 2 ? c0 : a.I + c0) + (rbi & 1) * 16;
    const int nb = row_first >> 4;
    const int nk_h = nk / 2, k0c = kh * nk_h, nk_w = kh ? nk - nk_h : nk_h;
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.W13 + (long long)eg * a.stride_we, (uint32_t)a.stride_we);
    const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.S13 + (long long)eg * a.stride_se, (uint32_t)a.stride_se);
    const uint32_t wv = (uint32_t)wtile_off<TILED>(nb, k0c, nk, Kh, lane), sv = (uint32_t)stile_off<TILED>(nb, k0c, nk, Ks, lane);
    const int ws = TILED ? 1024 : 64, ss = TILED ? 64 : 4;
    const int col = lane & 15, kb = lane >> 4;
    uint8_t* lds_s = smem + a.rows * LS;
    v4i A[PF];
    int SA[PF];
    const uint8_t* xl;
    const uint8_t* xsl;
    v4f acc;
    auto load = [&](int slot, int kc) {
        A[slot] = buffer_load_tile(wr, wv, (uint32_t)(kc * ws));
        SA[slot] = buffer_load_byte(sr, sv, (uint32_t)(kc * ss));
    };
    auto use = [&](int slot) {
        const v4i b0 = *(const v4i*)(xl);
        const v4i b1 = *(const v4i*)(xl + 64);
        const int sb = *xsl;
        xl += 128;
        xsl += 4;
        acc = mfma_fp4w_fp8x(v8i{A[slot].x, A[slot].y, A[slot].z, A[slot].w, 0, 0, 0, 0},
                             v8i{b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w}, acc, SA[slot], sb);
    };
    // Activation rows base .. base + mp - 1 of the group -> E4M3 codes + E8M0 bytes in LDS. Two lanes per
    // 32-value group, 16 values (2 x 16 bytes) each; a lane pair is always active together.
    auto stage = [&](int base, int mp) {
        const int per_row = Ks * 2;
#pragma unroll 1
        for (int i = tid; i < mp * per_row; i += blockDim.x) {
            const int r = i / per_row, q = i - r * per_row;
            const uint16_t* src = a.x + (long long)s_tok[base + r] * a.ldx + q * 16;
            const v4i r0 = *(const v4i*)src, r1 = *(const v4i*)(src + 8);
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
            for (int j = 0; j < 4; ++j) {
                cw[j] = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) cw[j] |= fq8_code(f[4 * j + b], e) << (8 * b);
            }
            *(v4i*)(smem + r * LS + q * 16) = v4i{(int)cw[0], (int)cw[1], (int)cw[2], (int)cw[3]};
            if ((q & 1) == 0) lds_s[r * Ks + (q >> 1)] = (uint8_t)(e + 127);
        }
    };
    // B columns: pass token col (columns past the pass read row 0; their results are not used)
    auto reset = [&](int mp) {
        const int brow = col < mp ? col : 0;
        xl = smem + brow * LS + k0c * 128 + kb * 16;
        xsl = lds_s + brow * Ks + k0c * 4 + kb;
        acc = v4f{0.f, 0.f, 0.f, 0.f};
    };
    // SwiGLU epilogue: half-wave i handles pass token i; lane c of it handles column c0 + c
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

    // One pass: LDS holds every token of the group (at most M when a token's expert ids are distinct, as the
    // gate guarantees; members past a.rows, possible only with repeated ids, are not computed). The weight
    // tiles go out first; quantising the activations into LDS overlaps their latency.
    const int mp0 = min(a.rows, mg);
    pipeline_start<PF>(nk_w, load);
    stage(0, mp0);
    __syncthreads();
    reset(mp0);
    pipeline_finish<PF>(nk_w, load, use);
    epilogue(0, mp0);
}

extern "C" int dsv41_moe_decode_up(const float* logits, long long ldl, const float* bias, float temp, float route_scale, int score_func,
                                   int norm, const int* eid_in, const float* wt_in, int M, int topk, int E, const uint16_t* x,
                                   long long ldx, const uint8_t* W13, long long stride_we, const uint8_t* S13, long long stride_se,
                                   int tiled, int H, int I, float limit, uint8_t* hc, long long ldhc, uint8_t* hs, long long ldhs,
                                   int* eid_out, float* wt_out, int* grp_expert, int* grp_start, int* tok_sorted, float* wt_sorted,
                                   void* stream) {
    if ((!logits && (!eid_in || !wt_in)) || !x || !W13 || !S13 || !hc || !hs || !grp_expert || !grp_start || !tok_sorted || !wt_sorted)
        return DSV41_EINVAL;
    if (M < 1 || M > UP_MAXM || topk < 1 || topk > UP_MAXK || topk > E || E < 1 || E > UP_MAXE || score_func < 0 || score_func > 2)
        return DSV41_EINVAL;
    if (H <= 0 || (H & 255) || I <= 0 || (I & 31) || ldx < H || (ldx & 7) || (((uintptr_t)x) & 15) || (logits && ldl < E)) return DSV41_EINVAL;
    // one expert's weights must be addressable with 32-bit offsets, and hold 2 I rows of H / 2 bytes
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll ||
        stride_we < (long long)2 * I * (H / 2) || stride_se < (long long)2 * I * (H / 32)) return DSV41_EINVAL;
    // LDS holds the quantised activations of every token of a group: at most M rows
    const size_t row_bytes = (size_t)(H + 16) + (size_t)(H / 32);
    const int rows = M;
    if (rows * row_bytes > UP_MAX_LDS) return DSV41_EINVAL;
    DecodeUpArgs a{logits, ldl, bias, temp, route_scale, score_func, norm, eid_in, wt_in, M, topk, E, rows, x, ldx, W13, stride_we, S13,
                   stride_se, H, I, limit, hc, ldhc, hs, ldhs, eid_out, wt_out, grp_expert, grp_start, tok_sorted, wt_sorted};
    const size_t lds = rows * row_bytes;
    const dim3 grid(I / 32, M * topk), block(UP_WAVES * 64);
    hipStream_t st = (hipStream_t)stream;
#define UP_LAUNCH(T, PER)                                                                                         \
    do {                                                                                                      \
        if (lds > 64 * 1024) {                                                                                \
            const hipError_t e = hipFuncSetAttribute((const void*)moe_decode_up_kernel<T, 8, PER>,             \
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);    \
            if (e != hipSuccess) return (int)e;                                                               \
        }                                                                                                     \
        moe_decode_up_kernel<T, 8, PER><<<grid, block, lds, st>>>(a);                                         \
    } while (0)
    if (E <= 256) { if (tiled) UP_LAUNCH(1, 4); else UP_LAUNCH(0, 4); }
    else { if (tiled) UP_LAUNCH(1, 8); else UP_LAUNCH(0, 8); }
#undef UP_LAUNCH
    return (int)hipGetLastError();
}
