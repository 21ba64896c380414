// Grouped FP4 expert GEMV/GEMM on gfx950 block-scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4).
//
// The weights are consumed as stored: E2M1 nibbles and their E8M0 bytes go straight into the MFMA A operand
// and its scale operand, so no instruction decodes a weight. The activations are FP8 E4M3 codes with E8M0
// bytes per 32 (what fake_quant_fp8 / swiglu_quant produce, exactly), fed as the B operand. One MFMA consumes
// a 16-row x 128-k weight tile = 1 KiB; both supported layouts make that tile one contiguous 1 KiB block
// (tile_fp4) or 16 contiguous 64 B row pieces (row-major), so every wave-wide weight load is fully used.
//
// Kernels:
//  fp4_grouped_kernel  out[p, n] = wt[p] * sum_k x[pair_tok[p], k] * deq(W[e_g])[n, k]  for pairs p of group g
//                      (cukern.fp4_gemm_tc / fp4_gemv_pairs / moe_kernels.grouped_fp4_gemm semantics,
//                      cukern.py:60-77, 238-276; moe_kernels.py:127-151). One wave = one (group, 16-row block);
//                      up to 16*NCH pairs share each weight tile (one MFMA per 16 pairs).
//  moe_down_sum_kernel y[t, n] = sum over groups g, pairs p of g with token t: h_p . deq(W2[e_g])[n, :]
//                      (decode w2 + the fixed per-token sum of decode.py:316-335 / fused2.py:490-495): the
//                      B column is the token, so all experts of a token accumulate in one MFMA accumulator and
//                      every selected expert's w2 is read once. Optional epilogue: bf16(y + shared-expert ys).
#include "common.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v8i widen(v4i a) { return v8i{a.x, a.y, a.z, a.w, 0, 0, 0, 0}; }
__device__ __forceinline__ v8i join(v4i a, v4i b) { return v8i{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}; }

struct GroupedArgs {
    const uint8_t* W; long long stride_we;   // [E][N][K/2] packed E2M1 (expert stride in bytes)
    const uint8_t* S; long long stride_se;   // [E][N][K/32] E8M0
    int N, K;
    const uint8_t* xc; long long ldx;        // FP8 codes [x_rows][K], row stride in bytes
    const uint8_t* xs; long long ldxs;       // E8M0 [x_rows][K/32], row stride in bytes
    int x_rows;                              // pair_tok values outside [0, x_rows) contribute zeros
    const int* grp_expert; const int* grp_start; const int* pair_tok;
    int n_pairs;                             // group ranges are clamped to [0, n_pairs)
    float* out; long long ldo;               // fp32 [out_rows][ldo]
    int out_rows;                            // output rows outside [0, out_rows) are not written
    const int* out_row;                      // optional: output row of pair p (default p)
    const float* pair_wt;                    // optional per-pair factor
    int shard_start, shard_n, zero_out, min_tok, max_tok, vec_store;
    int accum;                               // 0 store, 1 add (distinct rows), 2 atomic add (rows may repeat)
    int lds_rows;                            // B_LDS: activation rows staged per pass (<= 16)
    // TERMS == 2: the second FP8 term of off-grid activations (dsv41_quant_fp8_split), same strides as xc / xs
    const uint8_t* xlc; const uint8_t* xls;
    const int* run_if;                       // optional: the launch does nothing when *run_if == 0
    // XB: the activations as bf16 rows (xb [x_rows][ldxb], 8-k permuted when xb_perm) instead of codes: the workgroup
    // splits its staged rows into the two FP8 terms itself (fp8_split16, the codes dsv41_quant_fp8_split writes)
    const uint16_t* xb; long long ldxb; int xb_perm;
};

// LDS row stride for staged activation codes: +16 bytes so 16 rows fall in different banks
__device__ __forceinline__ int lds_stride(int K) { return K + 16; }

// A lane offset past every buffer this file's descriptors cover (the entries keep their byte counts below it)
#define OOB 0xFFFFFFF0u

// One wave = one (group, 16-row block); 4 waves per workgroup on consecutive row blocks of one group. A pass
// covers up to 16 pairs of the group (one MFMA column each); larger groups take several passes.
// B_LDS: the pass's activation rows are staged once per workgroup in LDS and read from there, so the vector
// memory queue holds only weight tiles (PF in flight per wave); otherwise B is read from global memory
// (L1/L2-resident) with non-divergent loads. Lanes whose column has no pair read row 0: their output
// column is never stored.
// TERMS == 2 (with B_LDS): the lo term's rows are staged beside the hi rows, and a pass covers up to 8 pairs: MFMA column
// c < 8 is pair c's hi row, column c + 8 its lo row, so one MFMA per weight tile computes both terms and the epilogue
// adds lane c + 8's accumulator to lane c's. For FP8-grid activations the lo codes are +0, so column c + 8 holds signed
// zeros and the sum is the one-term result bit for bit; no flag is read.
// XB (with TERMS == 2): the rows arrive as bf16 and are split into the two terms while being staged, after the first
// weight tiles went out, so no quantiser launch precedes the GEMM (the same codes and bytes as dsv41_quant_fp8_split).
template <int TILED, int PF, int B_LDS, int NKC, int TERMS = 1, int XB = 0>
__global__ void __launch_bounds__(256) fp4_grouped_kernel(const GroupedArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    static_assert(TERMS == 1 || B_LDS, "the second term is staged in LDS");
    static_assert(!XB || TERMS == 2, "bf16 rows are split into two terms");
    if (a.run_if && __builtin_amdgcn_readfirstlane(*a.run_if) == 0) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nb = blockIdx.x * 4 + wave;
    const int g = blockIdx.y;
    const bool active = nb * 16 < a.N;
    // the group's pair range, clamped to the n_pairs pairs the tables hold
    const int p0 = min(max(a.grp_start[g], 0), a.n_pairs), p1 = min(max(a.grp_start[g + 1], p0), a.n_pairs);
    const int m = p1 - p0;
    if (m <= 0 || m < a.min_tok || m > a.max_tok) return;       // uniform over the workgroup
    const int col = lane & 15, kb = lane >> 4;
    const int row0 = nb * 16 + 4 * kb;   // this lane's 4 output rows
    const int ge = a.grp_expert[g];
    const int e = ge - a.shard_start;
    // W holds experts shard_start .. shard_start + shard_n - 1 (all of them when unsharded); a group of another
    // GPU's expert (cukern.py:244-246) is skipped and, with zero_out, its rows zeroed; padding (-1) is skipped
    if (ge < 0 || e < 0 || e >= a.shard_n) {
        if (ge >= 0 && active && a.zero_out && a.accum == 0)
            for (int q = p0 + col; q < p1; q += 16) {
                const long long orow = a.out_row ? a.out_row[q] : q;
                if (orow < 0 || orow >= a.out_rows) continue;
#pragma unroll
                for (int i = 0; i < 4; ++i) a.out[orow * a.ldo + row0 + i] = 0.f;
            }
        return;
    }
    const int K = a.K, nk = K >> 7, Kh = K >> 1, Ks = K >> 5;
    // the expert's weights and scales through buffer descriptors (base and byte count in scalar registers, a 32-bit
    // lane offset, the k step as a scalar offset): 4 VGPRs per tile in flight instead of 64-bit addresses per slot
    const __amdgpu_buffer_rsrc_t wr = buffer_rsrc(a.W + (long long)e * a.stride_we, (uint32_t)a.stride_we);
    const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.S + (long long)e * a.stride_se, (uint32_t)a.stride_se);

    const uint32_t wvo = (uint32_t)wtile_off<TILED>(nb, 0, nk, Kh, lane), svo = (uint32_t)stile_off<TILED>(nb, 0, nk, Ks, lane);
    const int ws = TILED ? 1024 : 64, ss = TILED ? 64 : 4;
    const int LS = lds_stride(K);
    uint8_t* lds_s = smem + (size_t)a.lds_rows * LS;
    // the lo term's staged rows and bytes start lo_off bytes further (16-byte aligned)
    const int lo_off = (a.lds_rows * (LS + Ks) + 15) & ~15;

    const int PW = B_LDS ? a.lds_rows : 16;   // pairs per pass: never more rows than the LDS holds (TERMS == 2: <= 8)
    const int pc = TERMS == 2 ? (col & 7) : col;         // the lane's pair column in the pass
    const int term_off = TERMS == 2 && col >= 8 ? lo_off : 0;   // and its term (TERMS == 2: columns 8-15 read the lo rows)
    v4i A[PF];
    int SA[PF];
    v4i B0[B_LDS ? 1 : PF], B1[B_LDS ? 1 : PF];
    int SB[B_LDS ? 1 : PF];
    for (int base = p0; base < p1; base += PW) {
        const int mp = min(PW, p1 - base);
        const int brow = pc < mp ? pc : 0;
        // a pair whose token row is outside [0, x_rows) reads row 0 here and stores zeros below (global B path);
        // the LDS path stages a zero row for it
        const int tk = a.pair_tok[base + brow];
        const bool tok_ok = tk >= 0 && tk < a.x_rows;
        // the global path's activation rows through buffer descriptors too (x_rows * ldx < 2^32 - 16, checked by the entry)
        const __amdgpu_buffer_rsrc_t xr = buffer_rsrc(a.xc, B_LDS ? 0u : (uint32_t)((long long)a.x_rows * a.ldx));
        const __amdgpu_buffer_rsrc_t xsr = buffer_rsrc(a.xs, B_LDS ? 0u : (uint32_t)((long long)a.x_rows * a.ldxs));
        const uint32_t xvo = (uint32_t)((long long)(tok_ok ? tk : 0) * a.ldx + kb * 16);
        const uint32_t xsvo = (uint32_t)((long long)(tok_ok ? tk : 0) * a.ldxs + kb);
        const uint8_t* xl = smem + term_off + brow * LS + kb * 16;
        const uint8_t* xsl = lds_s + term_off + brow * Ks + kb;
        v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
        auto load = [&](int slot, int kc) {
            // the pipeline issues up to PF loads past the last k-chunk (unconditionally, so no slot register is a phi):
            // they take the lane offset OOB with no scalar offset, past every descriptor's byte count (the entry bounds
            // those below OOB), so they return zeros without a memory access; they are never consumed
            const bool in = kc < nk;
            const uint32_t k = in ? (uint32_t)kc : 0u;
            A[slot] = buffer_load_tile(wr, in ? wvo : OOB, k * ws);
            SA[slot] = buffer_load_byte(sr, in ? svo : OOB, k * ss);
            if (!B_LDS) {
                const uint32_t xo = in ? xvo : OOB;
                B0[slot] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, xo, k * 128, 0));
                B1[slot] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xr, xo, k * 128 + 64, 0));
                SB[slot] = buffer_load_byte(xsr, in ? xsvo : OOB, k * 4);
            }
        };
        auto use = [&](int slot) {
            // B_LDS reads the k-chunk of this slot by counter: slots are consumed in k order
            if (B_LDS) {
                const v4i b0 = *(const v4i*)(xl);
                const v4i b1 = *(const v4i*)(xl + 64);
                const int sb = *xsl;
                xl += 128;
                xsl += 4;
                acc = mfma_fp4w_fp8x(widen(A[slot]), join(b0, b1), acc, SA[slot], sb);
            } else {
                acc = mfma_fp4w_fp8x(widen(A[slot]), join(B0[slot], B1[slot]), acc, SA[slot], SB[slot]);
            }
        };
        // the first weight tiles go out before the activations are staged: staging overlaps their latency
        if (active) pipeline_start<PF>(nk, load);
        if (B_LDS && XB) {
            __syncthreads();
            // stage rows base .. base+mp-1 from bf16: thread i takes 16 values (chunk v of row r), a 32-group's two chunks
            // on adjacent lanes (vpr is even, so a lane pair is in or out of the range together); every load of a round is
            // issued before the first split
            const int vpr = K >> 4;
            constexpr int U = 2;
            for (int i0 = threadIdx.x; i0 < mp * vpr; i0 += U * (int)blockDim.x) {
                v4i w0[U], w1[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int i = i0 + u * (int)blockDim.x;
                    const int r = i / vpr, v = i - r * vpr;
                    const int t = i < mp * vpr ? a.pair_tok[base + r] : -1;
                    const bool ok = t >= 0 && t < a.x_rows;
                    const uint16_t* src = a.xb + (long long)(ok ? t : 0) * a.ldxb + v * 16;
                    w0[u] = ok ? *(const v4i*)src : v4i{0, 0, 0, 0};
                    w1[u] = ok ? *(const v4i*)(src + 8) : v4i{0, 0, 0, 0};
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int i = i0 + u * (int)blockDim.x;
                    if (i < mp * vpr) {
                        const int r = i / vpr, v = i - r * vpr;
                        v4i hi, lo;
                        int e, e2;
                        fp8_split16(w0[u], w1[u], a.xb_perm, hi, lo, e, e2);
                        *(v4i*)(smem + r * LS + v * 16) = hi;
                        *(v4i*)(smem + lo_off + r * LS + v * 16) = lo;
                        if ((v & 1) == 0) {
                            lds_s[r * Ks + (v >> 1)] = (uint8_t)(e + 127);
                            lds_s[lo_off + r * Ks + (v >> 1)] = (uint8_t)(e2 + 127);
                        }
                    }
                }
            }
            __syncthreads();
        } else if (B_LDS) {
            __syncthreads();
            {
                // stage rows base .. base+mp-1, both terms: each thread issues all loads of a round (16-byte code vectors,
                // 4-byte E8M0 words) before its first LDS store, so staging costs one memory round trip per round rather
                // than one per array
                const int vpr = K >> 4, wpr = K >> 7;   // code vectors and scale words per row (wpr <= vpr)
                constexpr int U = 2;                     // items per thread per round
                for (int i0 = threadIdx.x; i0 < mp * vpr; i0 += U * (int)blockDim.x) {
                    v4i hv[U], lv[U];
                    uint32_t hw[U], lw[U];
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int i = i0 + u * (int)blockDim.x;
                        const int r = i / vpr, v = i - r * vpr;
                        const int t = i < mp * vpr ? a.pair_tok[base + r] : -1;
                        const bool ok = t >= 0 && t < a.x_rows;
                        hv[u] = ok ? *(const v4i*)(a.xc + (long long)t * a.ldx + v * 16) : v4i{0, 0, 0, 0};
                        if (TERMS == 2) lv[u] = ok ? *(const v4i*)(a.xlc + (long long)t * a.ldx + v * 16) : v4i{0, 0, 0, 0};
                        const int rs = i / wpr, ws_ = i - rs * wpr;
                        const int ts = i < mp * wpr ? a.pair_tok[base + rs] : -1;
                        const bool oks = ts >= 0 && ts < a.x_rows;
                        hw[u] = oks ? *(const uint32_t*)(a.xs + (long long)ts * a.ldxs + 4 * ws_) : 0x7F7F7F7Fu;
                        if (TERMS == 2) lw[u] = oks ? *(const uint32_t*)(a.xls + (long long)ts * a.ldxs + 4 * ws_) : 0x7F7F7F7Fu;
                    }
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        const int i = i0 + u * (int)blockDim.x;
                        if (i < mp * vpr) {
                            const int r = i / vpr, v = i - r * vpr;
                            *(v4i*)(smem + r * LS + v * 16) = hv[u];
                            if (TERMS == 2) *(v4i*)(smem + lo_off + r * LS + v * 16) = lv[u];
                        }
                        if (i < mp * wpr) {
                            const int rs = i / wpr, ws_ = i - rs * wpr;
                            *(uint32_t*)(lds_s + rs * Ks + 4 * ws_) = hw[u];
                            if (TERMS == 2) *(uint32_t*)(lds_s + lo_off + rs * Ks + 4 * ws_) = lw[u];
                        }
                    }
                }
            }
            __syncthreads();
        }
        if (!active) continue;
        pipeline_finish<PF, B_LDS != 0, true>(nk, load, use);
        if (TERMS == 2) {   // pair column pc: its hi sum (lane pc) plus its lo sum (lane pc + 8)
            acc.x += __shfl_xor(acc.x, 8);
            acc.y += __shfl_xor(acc.y, 8);
            acc.z += __shfl_xor(acc.z, 8);
            acc.w += __shfl_xor(acc.w, 8);
        }
        const long long orow = a.out_row ? (long long)a.out_row[base + brow] : (long long)(base + brow);
        if ((TERMS == 1 || col < 8) && pc < mp && orow >= 0 && orow < a.out_rows) {
            const int q = base + pc;
            const float f = a.pair_wt ? a.pair_wt[q] : 1.f;
            float* o = a.out + orow * a.ldo + row0;
            const v4f v = (B_LDS || tok_ok) ? acc * f : v4f{0.f, 0.f, 0.f, 0.f};
            if (a.accum == 2) {
                atomicAdd(o + 0, v.x); atomicAdd(o + 1, v.y); atomicAdd(o + 2, v.z); atomicAdd(o + 3, v.w);
            } else if (a.accum == 1) {
                o[0] += v.x; o[1] += v.y; o[2] += v.z; o[3] += v.w;
            } else if (a.vec_store) {
                *(v4f*)o = v;
            } else {
                o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------ decode w2 + sum
struct DownSumArgs {
    const uint8_t* W; long long stride_we;
    const uint8_t* S; long long stride_se;
    int N, K;                                 // N = hidden (output rows), K = intermediate
    const uint8_t* hc; long long ldh;         // FP8 codes of h, pairs in expert-sorted order; row `zero_row` is 0
    const uint8_t* hs; long long ldhs;
    int zero_row;                             // an all-zero row of hc / hs (absent token columns read it)
    const int* grp_expert; const int* grp_start; const int* tok_sorted;
    int n_slots;                              // group slots to scan (= pairs); unused slots have expert -1
    int M;                                    // tokens (<= 16)
    float* y; long long ldy;                  // optional fp32 [M][N] routed sum
    const uint16_t* ys; long long ldys;       // optional bf16 shared-expert output
    uint16_t* yb; long long ldyb;             // optional bf16 [M][N] = bf16(y + ys)
    int shard_start, shard_n;
    // SH: the bf16 shared expert's down projection in the same launch. gus: its bf16 gate/up [M][ldgus] (the up
    // launch's output); each workgroup turns it into h_s = fq8(bf16(silu(min(g, L)) * clamp(u, +-L))) in LDS and adds
    // bf16(h_s . Ws2[rows]^T) (Ws2 bf16 [N][ldws2]) to y before the bf16 rounding; ys_out (optional) receives it
    const uint16_t* gus; long long ldgus; const uint16_t* Ws2; long long ldws2; float limit; uint16_t* ys_out; long long ldyso;
    int sh_tiled;   // Ws2 in 16 x 32 tiles of 1 KiB ([N/16][K/32][16][32], ldws2 = K) instead of row-major
    // optional hyper-connection post mix in the epilogue (fused2.hc_post2_, fused2.py:476-508): with x = bf16(y + ys),
    // each of the 4 residual streams r_i (bf16, token t's streams at hres + 4 N t + N i) <- bf16(post[t][i] x +
    // sum_j comb[t][j][i] r_j), in place (post fp32 [M][4], comb fp32 [M][4][4])
    uint16_t* hres; const float* hpost; const float* hcomb;
    // SH == 2: Ws2 is FP8 E4M3 (read as bytes, ldws2 = K bytes per row) in the w8 tile order [N/16][K/64][4][16][16 B],
    // with E8M0 scales Ss2 [N/32][ldss2] per 32 x 32 block
    const uint8_t* Ss2; long long ldss2;
};

#define DS_MAX_SLOTS 256
#define DS_WAVES 8
#define DS_HV 8          // H_LDS: h code vectors (16 bytes) per thread: 60 KiB of rows / 512 threads, rounded up
#define DS_HS 4          // H_LDS: h E8M0 bytes per thread (rows * K / 32 <= 2048 whenever the rows fit 60 KiB)
#define DS_HV_SH 4       // SH: the same with the shared expert's registers beside them (at most 32 KiB of h rows)
#define DS_SHC 7         // SH: the shared expert's 32-k chunks per wave (K / 32 <= 8 DS_SHC)
#define DS_SHC8 5        // SH == 2 (FP8): its 64-k chunks per wave (K / 64 <= 8 DS_SHC8)
#define DS_HS_SH 2
#ifndef DS_PF_SH
#define DS_PF_SH 4       // SH: weight tiles in flight per wave (12: the bf16 shared-expert layer 2.2 us slower, FP8 1.9)
#endif
#define DS_SCG 2         // SCL: groups per wave whose weight scales are staged in LDS
#define DS_SCW 2048      // SCL: LDS bytes per wave for them (<= 32 k-chunks of 64 bytes)
                         // SCL == 2: the current group's weight scales (<= 1 KiB) + its 16 h scale rows (64 bytes each)
#define DS_GUV 2         // SH: 16-byte vectors of the shared expert's gate/up rows per thread (M * 2K * 2 <= 16 * 512 * DS_GUV)

// One workgroup per 16-row block of the output; its 8 waves split the selected experts (group slots g = wave,
// wave + 8, ...), each accumulating sum over its experts and k of W2[e] . h in one MFMA accumulator whose
// column t is token t; a token absent from a group reads the zero row. The partial accumulators are summed in
// a fixed order through LDS. A wave walks its (group, k-chunk) space with a scalar iterator, so the weight
// pipeline runs across expert boundaries without branches.
// Prologue: every table is fetched in one round trip. H_LDS: all h rows (+ the zero row) are staged in LDS. Their
// loads go out right behind the tables and ahead of the weight tiles: loads complete in issue order, so the LDS copy
// of h then waits for h alone, not for the tiles; the tiles (their addresses need only the group experts) follow as
// soon as the tables are in. SCL (at most DS_SCG groups per wave, <= 32 k-chunks): each wave's weight scales are
// fetched with a few wide loads ahead of its tiles and read from LDS per k-step, instead of a one-byte load per
// lane with every tile (those cost the load unit as much time as the tiles).
// SCL == 2 (h rows from global, <= 16 k-chunks): a group's weight scales and the h scales of its 16 rows are fetched
// with one wide load each when the producer enters the group, into registers of the tile slot that starts it; the
// consumer copies them into the wave's LDS region when it reaches that tile and reads its bytes there per k-step.
// Three loads per tile remain (weights, two h vectors) instead of five.
// SH (with H_LDS): the bf16 shared expert's down projection for the same 16 rows. Its gate/up rows are loaded in the
// prologue with the h rows (16-byte vectors, staged in LDS where the end-of-kernel reduction buffers live), and h_s is
// built in LDS (bf16, [M][K + 8]) between the prologue's two barriers. Its 32-k chunks (16 rows x 64 bytes of Ws2 =
// 1 KiB per wave-load) are split over the 8 waves; a wave's chunks go out right behind its first routed tiles, into
// their own registers, and are consumed after the routed pipeline, in straight-line code, so the routed pipeline runs
// exactly as without the shared expert (mixing the two kinds in one tile loop costs its exact wait counts).
template <int TILED, int PF, int NKC, int H_LDS, int SCL, int SH = 0>
__global__ void __launch_bounds__(DS_WAVES * 64, H_LDS ? 4 : 2) moe_down_sum_kernel(const DownSumArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ short s_pair[DS_MAX_SLOTS][16];        // pair row of token t in group slot g (zero row if absent)
    __shared__ int s_start[DS_MAX_SLOTS + 1];
    __shared__ short s_tok[DS_MAX_SLOTS];
    // the waves' accumulators for the final reduction (SH: then the shared expert's after them); SH also stages the
    // shared expert's gate/up rows here during the prologue, long before the reduction
    __shared__ v4f s_red_all[SH ? 2 * DS_WAVES : DS_WAVES][64];
    v4f (*s_red)[64] = s_red_all;
    __shared__ __align__(16) uint8_t s_sc[SCL ? DS_WAVES * DS_SCW : 16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nb = blockIdx.x;
    const int K = a.K, Ks = K >> 5, LS = K + 16;
    const int n_slots = a.n_slots;
    // every kernel argument the prologue needs is read in one batch here (the empty asm consumes them), rather
    // than in one scalar round trip per first use
    __asm__ volatile("" ::"s"(a.W), "s"(a.stride_we), "s"(a.S), "s"(a.stride_se), "s"(K), "s"(n_slots), "s"(a.grp_expert),
                     "s"(a.grp_start), "s"(a.tok_sorted), "s"(a.shard_start), "s"(a.shard_n), "s"(a.hc), "s"(a.ldh), "s"(a.zero_row),
                     "s"(a.hs), "s"(a.ldhs));

    // ---- one round trip: this wave's group experts (slot wave + 8 j in lane j), the group starts, the tokens.
    // The loads are unconditional (indices clamped, results masked), so the kernel-argument loads they need go
    // out in one batch at entry instead of one round trip per guarded block.
    const int gslot = wave + DS_WAVES * lane;
    const bool gvalid = lane < DS_MAX_SLOTS / DS_WAVES && gslot < n_slots;
    const int st_l = a.grp_start[min(tid, n_slots)];        // n_slots + 1 entries
    int ge = -1, tk_l = 0;
    if (n_slots > 0) {                                        // uniform
        ge = a.grp_expert[min(gslot, n_slots - 1)];
        tk_l = a.tok_sorted[min(tid, n_slots - 1)];
    }
    // H_LDS: h rows 0 .. zero_row into registers now (buffer loads: a vector past the rows reads 0 and is not
    // stored); waves past the last vector issue none
    const int vpr = K >> 4, n_hv = (a.zero_row + 1) * vpr, n_hs = (a.zero_row + 1) * Ks;
    constexpr int NHV = SH ? DS_HV_SH : DS_HV, NHS = SH ? DS_HS_SH : DS_HS;
    v4i HV[H_LDS ? NHV : 1];
    int HS[H_LDS ? NHS : 1];
    if (H_LDS) {
        const __amdgpu_buffer_rsrc_t hr = buffer_rsrc(a.hc, (uint32_t)((long long)a.zero_row * a.ldh + K));
        const __amdgpu_buffer_rsrc_t hsr = buffer_rsrc(a.hs, (uint32_t)((long long)a.zero_row * a.ldhs + Ks));
#pragma unroll
        for (int i = 0; i < NHV; ++i) {
            const int idx = i * DS_WAVES * 64 + tid, r = idx / vpr, v = idx - r * vpr;
            if (i * DS_WAVES * 64 + wave * 64 < n_hv)   // wave-uniform
                HV[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(hr, idx < n_hv ? (uint32_t)(r * a.ldh + v * 16) : 0xFFFFFFF0u, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < NHS; ++i) {
            const int idx = i * DS_WAVES * 64 + tid, r = idx / Ks, v = idx - r * Ks;
            if (i * DS_WAVES * 64 + wave * 64 < n_hs)
                HS[i] = buffer_load_byte(hsr, idx < n_hs ? (uint32_t)(r * a.ldhs + v) : 0xFFFFFFF0u, 0);
        }
    }
    // SH: the shared expert's gate/up rows (M rows of 2K bf16 = 4K bytes each), 16-byte vectors, loaded with the h rows
    // (past the rows the offset is beyond the descriptor: zeros, no fetch)
    const int gvr = SH ? (K >> 2) : 0;                  // vectors per row
    const int n_gv = SH ? a.M * gvr : 0;
    v4i GV[SH ? DS_GUV : 1];
    if (SH) {
        const __amdgpu_buffer_rsrc_t gr = buffer_rsrc(a.gus, (uint32_t)((long long)(a.M - 1) * a.ldgus * 2 + 4 * K));
#pragma unroll
        for (int i = 0; i < DS_GUV; ++i) {
            const int idx = i * DS_WAVES * 64 + tid, t = idx / (gvr > 0 ? gvr : 1), v = idx - t * gvr;
            GV[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                gr, idx < n_gv ? (uint32_t)(t * a.ldgus * 2 + v * 16) : 0xFFFFFFF0u, 0, 0));
        }
    }
    int e = gvalid && ge >= 0 ? ge - a.shard_start : -1;
    if (e >= a.shard_n) e = -1;
    const int st = tid <= n_slots ? st_l : 0, tk = tid < n_slots ? tk_l : 0;
    const unsigned long long vmask = __ballot(e >= 0);   // this wave's valid groups

    const int col = lane & 15, kb = lane >> 4;
    const int nk = NKC > 0 ? NKC : (K >> 7), Kh = K >> 1;
    const uint32_t w0 = (uint32_t)wtile_off<TILED>(nb, 0, nk, Kh, lane), s0 = (uint32_t)stile_off<TILED>(nb, 0, nk, Ks, lane);
    const int ws = TILED ? 1024 : 64, ss = TILED ? 64 : 4;
    const int total = __popcll(vmask) * nk;
    // producer iterator (load order = consume order): valid-lane mask, k-chunk, expert
    unsigned long long pm = vmask;
    int pkc = 0;
    long long pe = pm ? __builtin_amdgcn_readlane(e, (int)__builtin_ctzll(pm)) : 0;
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    v4i A[PF], B0[H_LDS ? 1 : PF], B1[H_LDS ? 1 : PF];
    int SA[PF], SB[H_LDS ? 1 : PF];
    const uint8_t* hs_l = smem + (size_t)(a.zero_row + 1) * LS;
    // !H_LDS: the lane's h row (global) of the producer's current group, set at group boundaries
    const uint8_t* phb = a.hc;
    const uint8_t* phs = a.hs;
    // SCL == 2: lane (col, kb) fetches 16 bytes of its row's h scales at min(16 kb, Ks - 16) (the row's Ks bytes,
    // Ks >= 16, overlaps repeat the same bytes); the descriptor ends at the zero row's last scale
    constexpr bool GS = SCL == 2;
    const int gsb = min(kb * 16, Ks - 16);
    uint32_t pso = 0;
    auto prod_rows = [&]() {
        const long long q = pm ? s_pair[wave + DS_WAVES * (int)__builtin_ctzll(pm)][col] : a.zero_row;
        phb = a.hc + q * a.ldh + kb * 16;
        phs = a.hs + q * a.ldhs + kb;
        if (GS) pso = (uint32_t)(q * a.ldhs + gsb);
    };
    // SCL == 2: the group scale registers of each tile slot (written only by the tile that starts a group)
    v4i GA[GS ? PF : 1], GB[GS ? PF : 1];
    auto load = [&](int slot, int) {
        // one expert's tiles through a buffer descriptor: scalar base, 32-bit lane offset, scalar k offset
        // once the wave's groups are exhausted (H_LDS issues its first PF tiles unconditionally) the descriptor is
        // empty: the load returns zeros without touching memory, and the slot is never consumed
        const uint32_t wb = pm ? (uint32_t)a.stride_we : 0u, sbn = pm ? (uint32_t)a.stride_se : 0u;
        if (GS && pkc == 0) {
            // the producer enters a group: its weight scales (16 rows x nk k-chunks) and its rows' h scales, older
            // than the tile loads of this slot, so the wait for the slot covers them
            const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.S + pe * a.stride_se, sbn);
            if (TILED) {   // contiguous: 64 nb nk .. + 64 nk
                GA[slot] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                    sr, lane * 16 < nk * 64 ? (uint32_t)(nb * nk * 64 + lane * 16) : 0xFFFFFFF0u, 0, 0));
            } else {       // one dword (4 k-blocks) per (row, k-chunk)
                int g[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int idx = 64 * i + lane, r = idx & 15, kc = idx >> 4;
                    g[i] = (int)__builtin_amdgcn_raw_buffer_load_b32(sr, kc < nk ? (uint32_t)((nb * 16 + r) * Ks + kc * 4) : 0xFFFFFFF0u, 0, 0);
                }
                GA[slot] = v4i{g[0], g[1], g[2], g[3]};
            }
            GB[slot] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                buffer_rsrc(a.hs, (uint32_t)((long long)a.zero_row * a.ldhs + Ks)), pso, 0, 0));
        }
        A[slot] = buffer_load_tile(buffer_rsrc(a.W + pe * a.stride_we, wb), w0, (uint32_t)(pkc * ws));
        if (!SCL) SA[slot] = buffer_load_byte(buffer_rsrc(a.S + pe * a.stride_se, sbn), s0, (uint32_t)(pkc * ss));
        if (!H_LDS) {
            B0[slot] = *(const v4i*)phb;
            B1[slot] = *(const v4i*)(phb + 64);
            if (!GS) SB[slot] = *phs;
            phb += 128;
            phs += 4;
        }
        if (++pkc == nk) {
            pkc = 0;
            pm &= pm - 1ull;
            pe = pm ? __builtin_amdgcn_readlane(e, (int)__builtin_ctzll(pm)) : 0;
            if (!H_LDS) prod_rows();
        }
    };
    // consumer iterator: the lane's h row pointers move along k and jump at group boundaries
    unsigned long long cm = vmask;
    int ckc = 0;
    const uint8_t* hb = smem;
    const uint8_t* hsb = hs_l;
    auto group_rows = [&]() {
        const int q = cm ? s_pair[wave + DS_WAVES * (int)__builtin_ctzll(cm)][col] : a.zero_row;
        hb = smem + q * LS + kb * 16;
        hsb = hs_l + q * Ks + kb;
    };
    // SCL: the wave's staged scales in consume order (group j of the wave at 64 nk j, k-chunk kc at 64 kc within it)
    const uint8_t* wscl = s_sc + (SCL ? wave * DS_SCW : 0) + col * 4 + kb;
    // SCL == 2: weight scale of (col, kb) at k-chunk kc: 64 kc + 4 col + kb; h scale: 1024 + 64 col + 4 kc + kb
    const uint8_t* gsw = s_sc + (GS ? wave * DS_SCW : 0);
    // SH: h_s rows in LDS after the h rows and their scales (bf16, row stride K + 8); lane (col, kb) reads token col's
    // k [32 c + 8 kb, +8) (columns past the tokens read token 0: unused)
    const int hss = (K + 8) * 2;
    uint8_t* const hsh = smem + (((size_t)(a.zero_row + 1) * LS + (size_t)(a.zero_row + 1) * Ks + 15) & ~(size_t)15);
    auto use = [&](int slot) {
        if (GS && ckc == 0) {
            // the consumer enters a group (the previous group's reads were issued before, and one wave's LDS
            // operations complete in order)
            uint8_t* w = s_sc + wave * DS_SCW;
            if (TILED) {
                if (lane * 16 < nk * 64) *(v4i*)(w + lane * 16) = GA[slot];
            } else {
                const int g[4] = {GA[slot].x, GA[slot].y, GA[slot].z, GA[slot].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int idx = 64 * i + lane, r = idx & 15, kc = idx >> 4;
                    if (kc < nk) *(int*)(w + kc * 64 + r * 4) = g[i];
                }
            }
            int* hw = (int*)(w + 1024 + col * 64 + gsb);   // 4-byte aligned: Ks % 4 == 0
            hw[0] = GB[slot].x; hw[1] = GB[slot].y; hw[2] = GB[slot].z; hw[3] = GB[slot].w;
        }
        if (H_LDS) {
            const v4i b0 = *(const v4i*)hb;
            const v4i b1 = *(const v4i*)(hb + 64);
            const int sb = *hsb;
            const int sa = SCL ? (int)*wscl : SA[slot];
            hb += 128;
            hsb += 4;
            if (SCL) wscl += 64;
            acc = mfma_fp4w_fp8x(widen(A[slot]), join(b0, b1), acc, sa, sb);
        } else {
            const int sa = GS ? (int)gsw[ckc * 64 + col * 4 + kb] : SA[slot];
            const int sb = GS ? (int)gsw[1024 + col * 64 + ckc * 4 + kb] : SB[slot];
            acc = mfma_fp4w_fp8x(widen(A[slot]), join(B0[slot], B1[slot]), acc, sa, sb);
        }
        if (++ckc == nk) {
            ckc = 0;
            cm &= cm - 1ull;
            if (H_LDS) group_rows();
        }
    };
    // SCL: the scales of the wave's first DS_SCG groups (16 rows x nk k-chunks each), older than every tile. A missing
    // group reads through an empty descriptor (zeros) and is never consumed.
    v4i SC[SCL == 1 ? (TILED ? DS_SCG : 4 * DS_SCG) : 1];
    if (SCL == 1) {
        unsigned long long m = vmask;
#pragma unroll
        for (int j = 0; j < DS_SCG; ++j) {
            const int lj = m ? (int)__builtin_ctzll(m) : 0;
            const long long ej = m ? __builtin_amdgcn_readlane(e, lj) : 0;
            const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.S + ej * a.stride_se, m ? (uint32_t)a.stride_se : 0u);
            if (TILED) {   // the group's bytes are contiguous: 64 nb nk .. + 64 nk
                SC[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                    sr, lane * 16 < nk * 64 ? (uint32_t)(nb * nk * 64 + lane * 16) : 0xFFFFFFF0u, 0, 0));   // past the group: no fetch
            } else {       // row r's bytes are contiguous: one dword (4 k-blocks) per (row, k-chunk)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int idx = 64 * i + lane, r = idx & 15, kc = idx >> 4;
                    SC[4 * j + i].x = (int)__builtin_amdgcn_raw_buffer_load_b32(sr, kc < nk ? (uint32_t)((nb * 16 + r) * Ks + kc * 4) : 0xFFFFFFF0u, 0, 0);
                }
            }
            m &= m - 1ull;
        }
    }
    if (H_LDS) {
        // the first PF tiles, unconditionally (pipeline_start's short-stream branch would leave the stores below
        // after a merge, where the wait count falls back to draining the tiles too)
#pragma unroll
        for (int i = 0; i < PF; ++i) {
            load(i, i);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    // SH: this wave's share of the shared expert's 32-k chunks (a contiguous range of at most DS_SHC), issued behind the
    // routed first tiles into their own registers and consumed after the routed pipeline (slots past the range read
    // zeros: offset beyond the descriptor)
    constexpr int NSH = SH == 2 ? DS_SHC8 : DS_SHC;
    const int shc = SH == 2 ? (K >> 6) : SH ? (K >> 5) : 0;
    const int sc0 = SH ? shc * wave / DS_WAVES : 0, n_sh = SH ? shc * (wave + 1) / DS_WAVES - sc0 : 0;
    v4i SW[SH ? NSH : 1];
    int SWS[SH == 2 ? NSH : 1];
    if (SH == 2) {
        // FP8: chunk c of row block nb is the 1 KiB tile at (nb K / 64 + c) 1024, lane l's 16 bytes at 16 l (row l % 16,
        // k 64 c + 16 (l / 16) .. +15); each lane's block scale byte travels with its tile (chunks past the range read an
        // in-range scale: finite, and the zero tile makes the product 0)
        const uint8_t* W2s = (const uint8_t*)a.Ws2;
        const __amdgpu_buffer_rsrc_t s2r = buffer_rsrc(W2s + (long long)nb * 16 * a.ldws2, (uint32_t)(16 * a.ldws2));
        const uint32_t wv2 = (uint32_t)lane * 16u + (uint32_t)sc0 * 1024u;
        const uint8_t* ssr = a.Ss2 + (long long)(nb >> 1) * a.ldss2 + (lane >> 5);
#pragma unroll
        for (int j = 0; j < NSH; ++j) {
            SW[j] = buffer_load_tile(s2r, j < n_sh ? wv2 : 0xFFFFFFF0u, (uint32_t)j * 1024u);
            SWS[j] = ssr[2 * min(sc0 + j, shc - 1)];
        }
    } else if (SH) {
        const __amdgpu_buffer_rsrc_t s2r = buffer_rsrc(a.Ws2 + (long long)nb * 16 * a.ldws2, (uint32_t)(16 * a.ldws2 * 2));
        // lane (col, kb)'s 16 bytes of chunk c: row col, k [32 c + 8 kb, +8); tiled: at 1024 c + 64 col + 16 kb
        const uint32_t cs = a.sh_tiled ? 1024u : 64u;
        const uint32_t wv2 = (uint32_t)(a.sh_tiled ? (lane & 15) * 64 + (lane >> 4) * 16 : ((lane & 15) * a.ldws2 + (lane >> 4) * 8) * 2) +
                             (uint32_t)sc0 * cs;
#pragma unroll
        for (int j = 0; j < DS_SHC; ++j) SW[j] = buffer_load_tile(s2r, j < n_sh ? wv2 : 0xFFFFFFF0u, (uint32_t)j * cs);
    }

    // ---- tables -> LDS (and h rows 0 .. zero_row when H_LDS: their loads are older than every tile), the wave's
    // weight scales (SCL), then the pair rows of every valid group
    if (tid <= n_slots) s_start[tid] = st;
    if (tid < n_slots) s_tok[tid] = (short)tk;
    if (H_LDS) {
#pragma unroll
        for (int i = 0; i < NHV; ++i) {
            const int idx = i * DS_WAVES * 64 + tid, r = idx / vpr, v = idx - r * vpr;
            if (i * DS_WAVES * 64 + wave * 64 < n_hv && idx < n_hv) *(v4i*)(smem + r * LS + v * 16) = HV[i];
        }
        uint8_t* hsw = smem + (size_t)(a.zero_row + 1) * LS;
#pragma unroll
        for (int i = 0; i < NHS; ++i) {
            const int idx = i * DS_WAVES * 64 + tid;
            if (i * DS_WAVES * 64 + wave * 64 < n_hs && idx < n_hs) hsw[idx] = (uint8_t)HS[i];
        }
    }
    if (SH) {
        uint8_t* gsh = (uint8_t*)s_red_all;
#pragma unroll
        for (int i = 0; i < DS_GUV; ++i) {
            const int idx = i * DS_WAVES * 64 + tid;
            if (idx < n_gv) *(v4i*)(gsh + idx * 16) = GV[i];
        }
    }
    if (SCL == 1) {
        uint8_t* w = s_sc + wave * DS_SCW;
#pragma unroll
        for (int j = 0; j < DS_SCG; ++j) {
            if (TILED) {
                if (lane * 16 < nk * 64) *(v4i*)(w + j * nk * 64 + lane * 16) = SC[j];
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int idx = 64 * i + lane, r = idx & 15, kc = idx >> 4;
                    if (kc < nk) *(int*)(w + (j * nk + kc) * 64 + r * 4) = SC[4 * j + i].x;
                }
            }
        }
    }
    __syncthreads();
    if (lane < DS_MAX_SLOTS / DS_WAVES && gslot < n_slots) {
#pragma unroll
        for (int t = 0; t < 16; ++t) s_pair[gslot][t] = (short)a.zero_row;
        if (e >= 0)
            for (int q = s_start[gslot]; q < s_start[gslot + 1]; ++q) s_pair[gslot][s_tok[q] & 15] = (short)q;
    }
    if (SH) {
        // h_s = fq8(bf16(silu(min(g, L)) * clamp(u, +-L))) per 32 columns (fused.py:284-306 without a routing weight:
        // the shared expert's swiglu_quant(gu, None, ...), model.py:410), stored as bf16 values; half-wave j takes the
        // 32-column groups j, j + 16, ... of every token
        const uint16_t* gsh = (const uint16_t*)s_red_all;
        const int shg = a.M * (K >> 5);
        for (int idx = tid >> 5; idx < shg; idx += 2 * DS_WAVES) {
            const int t = idx / (K >> 5), c = (idx - t * (K >> 5)) * 32 + (tid & 31);
            float gg = bf16_to_f32(gsh[t * 2 * K + c]), uu = bf16_to_f32(gsh[t * 2 * K + K + c]);
            if (a.limit > 0.f) {
                uu = fminf(fmaxf(uu, -a.limit), a.limit);
                gg = fminf(gg, a.limit);
            }
            const float h = bf16_round(gg * (1.0f / (1.0f + expf(-gg))) * uu);
            const int ex = fq8_exponent(wave_max32(fabsf(h)));
            *(uint16_t*)(hsh + (size_t)t * hss + c * 2) = (uint16_t)f32_to_bf16_bits(fq8_value(fq8_code(h, ex), ex));
        }
    }
    __syncthreads();
    if (H_LDS) {
        group_rows();
        if (total >= PF) {
            pipeline_finish<PF>(total, load, use);
        } else {   // every tile of the wave is in slots 0 .. total - 1 already
#pragma unroll
            for (int i = 0; i < PF; ++i)
                if (i < total) use(i);
        }
    } else {
        prod_rows();
        pipelined<PF>(total, load, use);
    }
    v4f acc_s = v4f{0.f, 0.f, 0.f, 0.f};
    if (SH == 2) {
        // FP8 chunks: lane (col, kb) takes token col's h_s k [64 c + 16 kb, +16) as two bf16 operands against the decoded
        // tile's lower and upper 8 k
        const uint8_t* hl = hsh + (size_t)(col < a.M ? col : 0) * hss + kb * 32;
#pragma unroll
        for (int j = 0; j < NSH; ++j) {
            const int c = min(sc0 + j, shc - 1);
            v8bf16_t lo, hi;
            decode16(SW[j], e8m0_to_f32((uint32_t)SWS[j]), lo, hi);
            const v4i b0 = *(const v4i*)(hl + c * 128), b1 = *(const v4i*)(hl + c * 128 + 16);
            acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, __builtin_bit_cast(v8bf, b0), acc_s, 0, 0, 0);
            acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, __builtin_bit_cast(v8bf, b1), acc_s, 0, 0, 0);
        }
    } else if (SH) {
        // the wave's shared-expert chunks: bf16 products of Ws2's 16 rows with h_s (lane (col, kb): token col's k
        // [32 c + 8 kb, +8); columns past the tokens read token 0, unused). Slots past the wave's range hold zeros and
        // read an in-range chunk of h_s (finite), so they add exactly 0.
        const uint8_t* hl = hsh + (size_t)(col < a.M ? col : 0) * hss + kb * 16;
#pragma unroll
        for (int j = 0; j < DS_SHC; ++j) {
            const int c = min(sc0 + j, shc - 1);
            const v4i b = *(const v4i*)(hl + c * 64);
            acc_s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, SW[j]), __builtin_bit_cast(v8bf, b), acc_s, 0, 0, 0);
        }
    }
    s_red[wave][lane] = acc;
    if (SH) s_red_all[DS_WAVES + wave][lane] = acc_s;
    __syncthreads();
    if (wave != 0) return;
    v4f sum = s_red[0][lane];
#pragma unroll
    for (int w = 1; w < DS_WAVES; ++w) sum += s_red[w][lane];
    v4f ssum = v4f{0.f, 0.f, 0.f, 0.f};
    if (SH) {
        ssum = s_red_all[DS_WAVES][lane];
#pragma unroll
        for (int w = 1; w < DS_WAVES; ++w) ssum += s_red_all[DS_WAVES + w][lane];
    }
    if (col >= a.M) return;
    const int row0 = nb * 16 + 4 * kb;
    if (a.y) {
        float* o = a.y + (long long)col * a.ldy + row0;
        o[0] = sum.x; o[1] = sum.y; o[2] = sum.z; o[3] = sum.w;
    }
    if (a.yb || a.hres || (SH && a.ys_out)) {
        const float v[4] = {sum.x, sum.y, sum.z, sum.w};
        const float sv[4] = {ssum.x, ssum.y, ssum.z, ssum.w};
        float xo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float t = v[i];
            if (SH) {   // the shared expert's output is a bf16 tensor (w8.py:102-103), added to the fp32 sum (model.py:590)
                const uint32_t yb16 = f32_to_bf16_bits(sv[i]);
                if (a.ys_out) a.ys_out[(long long)col * a.ldyso + row0 + i] = (uint16_t)yb16;
                t += bf16_to_f32(yb16);
            } else if (a.ys) {
                t += bf16_to_f32(a.ys[(long long)col * a.ldys + row0 + i]);
            }
            const uint32_t tb = f32_to_bf16_bits(t);
            xo[i] = bf16_to_f32(tb);
            if (a.yb) a.yb[(long long)col * a.ldyb + row0 + i] = (uint16_t)tb;
        }
        if (a.hres) {
            // the post mix for this lane's 4 columns of token col: all 4 streams read before any is written
            uint16_t* r = a.hres + (long long)col * 4 * a.N + row0;
            const float* pb = a.hpost + col * 4;
            const float* cb = a.hcomb + col * 16;
            float rv[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint2 u = *(const uint2*)(r + (long long)j * a.N);
                rv[j][0] = bf16_to_f32(u.x & 0xFFFFu); rv[j][1] = bf16_to_f32(u.x >> 16);
                rv[j][2] = bf16_to_f32(u.y & 0xFFFFu); rv[j][3] = bf16_to_f32(u.y >> 16);
            }
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                uint32_t o[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float acc = pb[s] * xo[c];
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc = fmaf(cb[j * 4 + s], rv[j][c], acc);
                    o[c] = f32_to_bf16_bits(acc);
                }
                *(uint2*)(r + (long long)s * a.N) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
            }
        }
    }
}

// ------------------------------------------------------------------------------------------ decode w2 + sum, split
// For token counts whose h rows do not fit LDS at once (dsv41_moe_down_sum_split; M > 4 at top-8): the expert groups
// are split into S runs of Q consecutive pair rows (a group belongs to the run holding its first row), and workgroup
// (rb, s) computes output rows 128 rb .. 128 rb + 127 (wave w: the 16-row block 8 rb + w) over run s's groups. The
// run's h rows (<= Q + M - 1 <= DX_ROWS - 1) and a zero row sit in LDS, so every 1 KiB weight tile costs one
// vector-memory instruction and its B operand (column t = token t) comes from LDS; a group's weight scales take one
// wide load when the wave enters it. part[s][t][n] receives the run's sums; down_reduce_kernel adds the S partials
// in run order and applies the epilogue of moe_down_sum_kernel.
#define DX_ROWS 32
#define DX_MAXG 32
#define DX_RUNS 16   // runs: ceil(n_slots / Q) <= 16 for n_slots <= 256, M <= 16

template <int TILED, int PF>
__global__ void __launch_bounds__(DS_WAVES * 64, 2) moe_down_split_kernel(const DownSumArgs a, float* __restrict__ part, int Q) {
    extern __shared__ __align__(16) uint8_t smem[];   // h codes [DX_ROWS][K + 16], then their E8M0 bytes [DX_ROWS][K / 32]
    __shared__ int s_gs[DS_MAX_SLOTS + 1];
    __shared__ int s_ge[DS_MAX_SLOTS];
    __shared__ short s_tok[DS_MAX_SLOTS];
    __shared__ int s_ex[DX_MAXG];                      // expert of the run's j-th group with an expert of this shard
    __shared__ signed char s_pair[DX_MAXG][16];        // LDS row of token t's pair in that group (DX_ROWS - 1: none)
    __shared__ int s_lo, s_hi;
    __shared__ __align__(16) uint8_t s_sc[DS_WAVES][1024];   // the wave's current group's weight scales
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rb = blockIdx.x, s = blockIdx.y;
    const int K = a.K, Ks = K >> 5, LS = K + 16, nk = K >> 7, Kh = K >> 1;
    const int n_slots = a.n_slots, M = a.M;
    const int nb = rb * 8 + wave;
    const int w0 = s * Q, w1 = w0 + Q;

    // ---- tables, one round trip
    for (int i = tid; i <= n_slots; i += DS_WAVES * 64) s_gs[i] = a.grp_start[i];
    for (int i = tid; i < n_slots; i += DS_WAVES * 64) {
        s_ge[i] = a.grp_expert[i];
        s_tok[i] = (short)a.tok_sorted[i];
    }
    if (tid == 0) {
        s_lo = DS_MAX_SLOTS;
        s_hi = -1;
    }
    __syncthreads();
    // the run's groups: first row in [w0, w1), expert id set (padding groups carry -1); they are consecutive
    for (int g = tid; g < n_slots; g += DS_WAVES * 64) {
        const int st = s_gs[g];
        if (s_ge[g] >= 0 && st >= w0 && st < w1 && s_gs[g + 1] > st) {
            atomicMin(&s_lo, g);
            atomicMax(&s_hi, g);
        }
    }
    __syncthreads();
    const int g0 = s_lo, g1 = s_hi + 1;   // g1 <= g0 when the run is empty
    const int ng = g1 > g0 ? g1 - g0 : 0;
    const int r0 = ng ? s_gs[g0] : 0, nr = ng ? s_gs[g1] - r0 : 0;   // <= Q + M - 1 rows

    // ---- the run's h rows into registers (16-byte vectors; past the rows the offset is beyond the descriptor: zeros)
    const int vpr = K >> 4;
    constexpr int NHV = (DX_ROWS * 2048 / 16 + DS_WAVES * 64 - 1) / (DS_WAVES * 64);   // K <= 2048
    constexpr int NHS = (DX_ROWS * 64 + DS_WAVES * 64 - 1) / (DS_WAVES * 64);            // K / 32 <= 64
    v4i HV[NHV];
    int HS[NHS];
    const __amdgpu_buffer_rsrc_t hr = buffer_rsrc(a.hc + (long long)r0 * a.ldh, (uint32_t)(nr > 0 ? (long long)(nr - 1) * a.ldh + K : 0));
    const __amdgpu_buffer_rsrc_t hsr = buffer_rsrc(a.hs + (long long)r0 * a.ldhs, (uint32_t)(nr > 0 ? (long long)(nr - 1) * a.ldhs + Ks : 0));
#pragma unroll
    for (int i = 0; i < NHV; ++i) {
        const int idx = i * DS_WAVES * 64 + tid, r = idx / vpr, v = idx - r * vpr;
        HV[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(hr, r < nr ? (uint32_t)(r * a.ldh + v * 16) : 0xFFFFFFF0u, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < NHS; ++i) {
        const int idx = i * DS_WAVES * 64 + tid, r = idx / Ks, v = idx - r * Ks;
        HS[i] = buffer_load_byte(hsr, r < nr ? (uint32_t)(r * a.ldhs + v) : 0xFFFFFFF0u, 0);
    }
    // the run's groups with an expert of this shard, compacted in order (wave 0: one lane per group), with their
    // token -> LDS row maps
    if (wave == 0) {
        const int g = g0 + lane;
        int e = -1;
        if (lane < ng) {
            e = s_ge[g] - a.shard_start;
            if (e >= a.shard_n) e = -1;
        }
        const unsigned long long vm = __ballot(e >= 0);
        if (e >= 0) {
            const int j = __popcll(vm & ((1ull << lane) - 1ull));
            s_ex[j] = e;
#pragma unroll
            for (int t = 0; t < 16; ++t) s_pair[j][t] = (signed char)(DX_ROWS - 1);
            for (int q = s_gs[g]; q < s_gs[g + 1]; ++q) s_pair[j][s_tok[q] & 15] = (signed char)(q - r0);
        }
        if (lane == 0) s_lo = __popcll(vm);   // the count, read back after the barrier
    }
    // h rows into LDS (row DX_ROWS - 1: zeros, scale byte 127)
    uint8_t* const hs_l = smem + (size_t)DX_ROWS * LS;
#pragma unroll
    for (int i = 0; i < NHV; ++i) {
        const int idx = i * DS_WAVES * 64 + tid, r = idx / vpr, v = idx - r * vpr;
        if (r < DX_ROWS - 1) *(v4i*)(smem + r * LS + v * 16) = HV[i];
    }
    for (int v = tid; v < vpr; v += DS_WAVES * 64) *(v4i*)(smem + (DX_ROWS - 1) * LS + v * 16) = v4i{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < NHS; ++i) {
        const int idx = i * DS_WAVES * 64 + tid, r = idx / Ks;
        if (r < DX_ROWS - 1) hs_l[idx] = (uint8_t)HS[i];
    }
    for (int v = tid; v < Ks; v += DS_WAVES * 64) hs_l[(DX_ROWS - 1) * Ks + v] = 127;
    __syncthreads();

    // ---- this wave's row block over the compacted groups: (group j, k-chunk kc) tiles through a PF-deep pipeline
    const int nv = __builtin_amdgcn_readfirstlane(s_lo);
    const int ex_l = lane < nv ? s_ex[lane] : 0;   // lane j holds group j's expert
    const int col = lane & 15, kb = lane >> 4;
    const uint32_t wv = (uint32_t)wtile_off<TILED>(nb, 0, nk, Kh, lane);
    const int ws = TILED ? 1024 : 64;
    const int total = nv * nk;
    // producer iterator: group pj, k-chunk pkc, expert pe
    int pj = 0, pkc = 0;
    long long pe = nv > 0 ? __builtin_amdgcn_readlane(ex_l, 0) : 0;
    v4i A[PF], GA[PF];
    auto load = [&](int slot, int) {
        const uint32_t wb = pj < nv ? (uint32_t)a.stride_we : 0u, sbn = pj < nv ? (uint32_t)a.stride_se : 0u;
        if (pkc == 0) {   // the producer enters a group: its weight scales for this row block, with the slot's tile
            const __amdgpu_buffer_rsrc_t sr = buffer_rsrc(a.S + pe * a.stride_se, sbn);
            if (TILED) {
                GA[slot] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                    sr, lane * 16 < nk * 64 ? (uint32_t)(nb * nk * 64 + lane * 16) : 0xFFFFFFF0u, 0, 0));
            } else {
                int gg[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int idx = 64 * i + lane, r = idx & 15, kc = idx >> 4;
                    gg[i] = (int)__builtin_amdgcn_raw_buffer_load_b32(sr, kc < nk ? (uint32_t)((nb * 16 + r) * Ks + kc * 4) : 0xFFFFFFF0u, 0, 0);
                }
                GA[slot] = v4i{gg[0], gg[1], gg[2], gg[3]};
            }
        }
        A[slot] = buffer_load_tile(buffer_rsrc(a.W + pe * a.stride_we, wb), wv, (uint32_t)(pkc * ws));
        if (++pkc == nk) {
            pkc = 0;
            ++pj;
            pe = pj < nv ? __builtin_amdgcn_readlane(ex_l, pj) : 0;
        }
    };
    // consumer iterator: group cj, k-chunk ckc; the lane's h row (token col) of the current group
    int cj = 0, ckc = 0;
    const uint8_t* hb = smem;
    const uint8_t* hsb = hs_l;
    auto group_rows = [&]() {
        const int q = cj < nv ? (int)s_pair[cj][col] : DX_ROWS - 1;
        hb = smem + q * LS + kb * 16;
        hsb = hs_l + q * Ks + kb;
    };
    group_rows();
    uint8_t* const wsc = s_sc[wave];
    v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
    auto use = [&](int slot) {
        if (ckc == 0) {   // the consumer enters a group: its weight scales into the wave's LDS region (k-chunk kc at 64 kc)
            if (TILED) {
                if (lane * 16 < nk * 64) *(v4i*)(wsc + lane * 16) = GA[slot];
            } else {
                const int gg[4] = {GA[slot].x, GA[slot].y, GA[slot].z, GA[slot].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int idx = 64 * i + lane, r = idx & 15, kc = idx >> 4;
                    if (kc < nk) *(int*)(wsc + kc * 64 + r * 4) = gg[i];
                }
            }
        }
        const v4i b0 = *(const v4i*)hb;
        const v4i b1 = *(const v4i*)(hb + 64);
        const int sb = *hsb;
        const int sa = wsc[ckc * 64 + col * 4 + kb];
        hb += 128;
        hsb += 4;
        acc = mfma_fp4w_fp8x(widen(A[slot]), join(b0, b1), acc, sa, sb);
        if (++ckc == nk) {
            ckc = 0;
            ++cj;
            group_rows();
        }
    };
    pipelined<PF>(total, load, use);
    if (col < M) {
        float* o = part + ((long long)s * M + col) * a.N + nb * 16 + 4 * kb;
        *(v4f*)o = acc;
    }
}

// y[t][n] = sum over the S runs of part[s][t][n] (run order), then the epilogue of moe_down_sum_kernel: the fp32 sum,
// bf16(y + ys), the hyper-connection post mix. One thread per 4 consecutive n.
__global__ void __launch_bounds__(256) down_reduce_kernel(const DownSumArgs a, const float* __restrict__ part, int S) {
    const int M = a.M, N = a.N, nq = N >> 2;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= M * nq) return;
    const int col = idx / nq, row0 = (idx - col * nq) * 4;
    // every run's partial in flight at once (S <= DX_RUNS), then summed in run order
    v4f pv[DX_RUNS];
#pragma unroll
    for (int s = 0; s < DX_RUNS; ++s)
        pv[s] = s < S ? *(const v4f*)(part + ((long long)s * M + col) * N + row0) : v4f{0.f, 0.f, 0.f, 0.f};
    v4f sum = pv[0];
#pragma unroll
    for (int s = 1; s < DX_RUNS; ++s)
        if (s < S) sum += pv[s];
    if (a.y) *(v4f*)(a.y + (long long)col * a.ldy + row0) = sum;
    if (a.yb || a.hres) {
        const float v[4] = {sum.x, sum.y, sum.z, sum.w};
        float xo[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float t = v[i];
            if (a.ys) t += bf16_to_f32(a.ys[(long long)col * a.ldys + row0 + i]);
            const uint32_t tb = f32_to_bf16_bits(t);
            xo[i] = bf16_to_f32(tb);
            if (a.yb) a.yb[(long long)col * a.ldyb + row0 + i] = (uint16_t)tb;
        }
        if (a.hres) {
            uint16_t* r = a.hres + (long long)col * 4 * N + row0;
            const float* pb = a.hpost + col * 4;
            const float* cb = a.hcomb + col * 16;
            float rv[4][4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint2 u = *(const uint2*)(r + (long long)j * N);
                rv[j][0] = bf16_to_f32(u.x & 0xFFFFu); rv[j][1] = bf16_to_f32(u.x >> 16);
                rv[j][2] = bf16_to_f32(u.y & 0xFFFFu); rv[j][3] = bf16_to_f32(u.y >> 16);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t o[4];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float acc = pb[q] * xo[c];
#pragma unroll
                    for (int j = 0; j < 4; ++j) acc = fmaf(cb[j * 4 + q], rv[j][c], acc);
                    o[c] = f32_to_bf16_bits(acc);
                }
                *(uint2*)(r + (long long)q * N) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
            }
        }
    }
}

// ------------------------------------------------------------------------------------------ C ABI
#define B_LDS_MAX_BYTES (48 * 1024)

template <int TILED, int B_LDS, int TERMS = 1, int XB = 0>
static void launch_grouped(const GroupedArgs& a, int G, size_t lds, hipStream_t st) {
    dim3 grid((unsigned)((a.N / 16 + 3) / 4), (unsigned)G);
    constexpr int PF = B_LDS ? DSV41_PF_UP : 8;
    fp4_grouped_kernel<TILED, PF, B_LDS, 0, TERMS, XB><<<grid, 256, lds, st>>>(a);
}

static void launch_grouped_any(const GroupedArgs& a, int G, bool use_lds, int terms, size_t lds, hipStream_t st, int tiled) {
    if (terms == 2) {
        if (tiled) launch_grouped<1, 1, 2>(a, G, lds, st); else launch_grouped<0, 1, 2>(a, G, lds, st);
    } else if (tiled) {
        if (use_lds) launch_grouped<1, 1>(a, G, lds, st); else launch_grouped<1, 0>(a, G, 0, st);
    } else {
        if (use_lds) launch_grouped<0, 1>(a, G, lds, st); else launch_grouped<0, 0>(a, G, 0, st);
    }
}

extern "C" int dsv41_fp4_grouped_gemm(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                                      int N, int K, const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, int x_rows,
                                      const uint8_t* xlc, const uint8_t* xls, const int* lo_flag,
                                      const int* grp_expert, const int* grp_start, int G, const int* pair_tok, int n_pairs,
                                      float* out, long long ldo, int out_rows, const int* out_row, const float* pair_wt, int accum,
                                      int max_tokens, int shard_start, int shard_n, int zero_out, int min_tok, int max_tok, void* stream) {
    if (!W || !S || !xc || !xs || !grp_expert || !grp_start || !pair_tok || !out) return DSV41_EINVAL;
    if (N <= 0 || (N & 15) || K <= 0 || (K & 127) || G < 0 || ldo < N || ldx < K || ldxs < K / 32 || max_tokens < 1) return DSV41_EINVAL;
    if (accum < 0 || accum > 2 || (ldx & 15) || (((uintptr_t)xc) & 15) || x_rows < 0 || n_pairs < 0 || out_rows < 0 || shard_n < 0)
        return DSV41_EINVAL;
    if ((long long)x_rows * ldx >= OOB || (long long)x_rows * ldxs >= OOB) return DSV41_EINVAL;   // 32-bit offsets, below OOB
    if ((ldxs & 3) || (((uintptr_t)xs) & 3) || (((uintptr_t)xls) & 3)) return DSV41_EINVAL;         // scale rows read as words
    // the second term comes whole (codes and scales; its flag optional) or not at all
    const int terms = xlc ? 2 : 1;
    if ((xlc != nullptr) != (xls != nullptr) || (lo_flag && !xlc) || (((uintptr_t)xlc) & 15)) return DSV41_EINVAL;
    // every expert W holds has N rows of K / 2 weight bytes and K / 32 scale bytes, within 32-bit buffer offsets
    if (stride_we < (long long)N * (K / 2) || stride_se < (long long)N * (K / 32) || stride_we >= OOB || stride_se >= OOB)
        return DSV41_EINVAL;
    if (G == 0 || n_pairs == 0) return 0;
    GroupedArgs a{W, stride_we, S, stride_se, N, K, xc, ldx, xs, ldxs, x_rows, grp_expert, grp_start, pair_tok, n_pairs, out, ldo, out_rows,
                  out_row, pair_wt, shard_start, shard_n, zero_out, min_tok, max_tok, 0, accum, 0, xlc, xls, nullptr};
    a.vec_store = ((ldo & 3) == 0 && (((uintptr_t)out) & 15) == 0) ? 1 : 0;
    hipStream_t st = (hipStream_t)stream;
    const int rows = max_tokens < 16 ? max_tokens : 16;
    const size_t lds1 = (size_t)rows * (K + 16) + (size_t)rows * (K / 32);
    const int rows2 = rows < 8 ? rows : 8;   // two terms: passes of up to 8 pairs (hi and lo in one MFMA's 16 columns)
    const size_t one2 = (size_t)rows2 * (K + 16) + (size_t)rows2 * (K / 32);
    const size_t lds2 = ((one2 + 15) & ~(size_t)15) + one2;
    if (terms == 2 && lds2 <= B_LDS_MAX_BYTES) {
        // both terms staged in LDS, one launch (lo_flag is not needed)
        a.lds_rows = rows2;
        launch_grouped_any(a, G, true, 2, lds2, st, tiled);
        return (int)hipGetLastError();
    }
    const bool use_lds = lds1 <= B_LDS_MAX_BYTES;
    a.lds_rows = use_lds ? rows : 0;
    a.xlc = a.xls = nullptr;
    launch_grouped_any(a, G, use_lds, 1, use_lds ? lds1 : 0, st, tiled);
    if (terms == 2) {
        // the activation rows do not fit LDS twice: the lo term as a second pass that adds into the same outputs; with
        // lo_flag it does nothing when no lo code is non-zero
        GroupedArgs b = a;
        b.xc = xlc;
        b.xs = xls;
        b.run_if = lo_flag;
        b.accum = accum == 2 ? 2 : 1;
        b.zero_out = 0;
        b.vec_store = 0;
        launch_grouped_any(b, G, use_lds, 1, use_lds ? lds1 : 0, st, tiled);
    }
    return (int)hipGetLastError();
}

// The same GEMM on bf16 activation rows x [x_rows][ldx] (elements; 8-k permuted when `permuted`): each workgroup splits
// the rows it stages into the two FP8 terms (the codes dsv41_quant_fp8_split writes), so the GEMM needs no quantiser
// launch before it. Only for passes whose two terms fit the LDS staging (min(max_tokens, 8) rows of K): otherwise
// DSV41_EINVAL, and the caller quantises first (dsv41_quant_fp8_split) and calls dsv41_fp4_grouped_gemm.
extern "C" int dsv41_fp4_grouped_gemm_bf16(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                                           int N, int K, const uint16_t* x, long long ldx, int x_rows, int permuted,
                                           const int* grp_expert, const int* grp_start, int G, const int* pair_tok, int n_pairs,
                                           float* out, long long ldo, int out_rows, const int* out_row, const float* pair_wt, int accum,
                                           int max_tokens, int shard_start, int shard_n, int zero_out, int min_tok, int max_tok,
                                           void* stream) {
    if (!W || !S || !x || !grp_expert || !grp_start || !pair_tok || !out) return DSV41_EINVAL;
    if (N <= 0 || (N & 15) || K <= 0 || (K & 127) || G < 0 || ldo < N || ldx < K || max_tokens < 1) return DSV41_EINVAL;
    if (accum < 0 || accum > 2 || (ldx & 7) || (((uintptr_t)x) & 15) || x_rows < 0 || n_pairs < 0 || out_rows < 0 || shard_n < 0)
        return DSV41_EINVAL;   // 16-byte row pieces
    if (stride_we < (long long)N * (K / 2) || stride_se < (long long)N * (K / 32) || stride_we >= OOB || stride_se >= OOB)
        return DSV41_EINVAL;
    const int rows2 = max_tokens < 8 ? max_tokens : 8;
    const size_t one2 = (size_t)rows2 * (K + 16) + (size_t)rows2 * (K / 32);
    const size_t lds2 = ((one2 + 15) & ~(size_t)15) + one2;
    if (lds2 > B_LDS_MAX_BYTES) return DSV41_EINVAL;
    if (G == 0 || n_pairs == 0) return 0;
    GroupedArgs a{W, stride_we, S, stride_se, N, K, nullptr, 0, nullptr, 0, x_rows, grp_expert, grp_start, pair_tok, n_pairs, out, ldo,
                  out_rows, out_row, pair_wt, shard_start, shard_n, zero_out, min_tok, max_tok, 0, accum, rows2, nullptr, nullptr, nullptr,
                  x, ldx, permuted ? 1 : 0};
    a.vec_store = ((ldo & 3) == 0 && (((uintptr_t)out) & 15) == 0) ? 1 : 0;
    hipStream_t st = (hipStream_t)stream;
    if (tiled) launch_grouped<1, 1, 2, 1>(a, G, lds2, st);
    else launch_grouped<0, 1, 2, 1>(a, G, lds2, st);
    return (int)hipGetLastError();
}

extern "C" int dsv41_moe_down_sum(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                                  int N, int K, const uint8_t* hc, long long ldh, const uint8_t* hs, long long ldhs, int zero_row,
                                  const int* grp_expert, const int* grp_start, const int* tok_sorted, int n_slots, int M,
                                  float* y, long long ldy, const uint16_t* ys, long long ldys, uint16_t* yb, long long ldyb,
                                  int shard_start, int shard_n, const uint16_t* gus, long long ldgus, const uint16_t* Ws2,
                                  long long ldws2, int sh_tiled, float limit, uint16_t* ys_out, long long ldyso, uint16_t* hres,
                                  const float* hpost, const float* hcomb, const uint8_t* Ss2, long long ldss2, void* stream) {
    if (!W || !S || !hc || !hs || !grp_expert || !grp_start || !tok_sorted || (!y && !yb && !ys_out && !hres)) return DSV41_EINVAL;
    if (hres && (!hpost || !hcomb || (((uintptr_t)hres) & 7))) return DSV41_EINVAL;
    // the fused shared expert: its gate/up (bf16 [M][ldgus], 2 K columns) and Ws2 (bf16 [N][ldws2], 16-byte row pieces,
    // 16-row blocks addressed with 32-bit offsets); it replaces a given ys
    const bool sh = Ws2 != nullptr;
    const bool sh_fp8 = sh && Ss2 != nullptr;   // FP8 E4M3 Ws2 in the w8 tile order (ldws2 = K bytes), E8M0 Ss2
    if (sh && (!gus || ys || ldgus < 2LL * K || ldws2 < K || (ldws2 & 7) || (((uintptr_t)Ws2) & 15) || 16 * ldws2 * 2 > 0xFFFFFFFFll ||
               (ldgus & 7) || (((uintptr_t)gus) & 15) || (sh_tiled && ldws2 != K) || (long long)M * 4 * K > 16LL * DS_WAVES * 64 * DS_GUV ||
               (long long)M * 4 * K > (long long)sizeof(v4f) * 2 * DS_WAVES * 64 || (ys_out && ldyso < N)))
        return DSV41_EINVAL;
    if (sh_fp8 && (!sh_tiled || ldws2 != K || (K & 63) || ldss2 < K / 32 || K / 64 > DS_SHC8 * DS_WAVES)) return DSV41_EINVAL;
    if (!sh && !y && !yb && !hres) return DSV41_EINVAL;
    // zero_row is kept in the kernel's 16-bit pair table
    if (N <= 0 || (N & 15) || K <= 0 || (K & 127) || n_slots < 0 || n_slots > DS_MAX_SLOTS || M < 1 || M > 16 || zero_row < 0 || zero_row > 32767)
        return DSV41_EINVAL;
    // one expert's weights are addressed with 32-bit offsets and hold N rows of K / 2 bytes
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll || stride_we < (long long)N * (K / 2) ||
        stride_se < (long long)N * (K / 32))
        return DSV41_EINVAL;
    if ((ldh & 15) || (((uintptr_t)hc) & 15) || ldh < K || ldhs < K / 32) return DSV41_EINVAL;
    if ((y && ldy < N) || (yb && ldyb < N) || (yb && ys && ldys < N)) return DSV41_EINVAL;
    DownSumArgs a{W, stride_we, S, stride_se, N, K, hc, ldh, hs, ldhs, zero_row, grp_expert, grp_start, tok_sorted, n_slots, M,
                  y, ldy, ys, ldys, yb, ldyb, shard_start, shard_n, gus, ldgus, Ws2, ldws2, limit, ys_out, ldyso, sh_tiled,
                  hres, hpost, hcomb, Ss2, ldss2};
    hipStream_t st = (hipStream_t)stream;
    // dynamic LDS: the h rows (codes, then their E8M0 bytes) and, with the shared expert, its bf16 h_s rows
    const size_t lds_h = (size_t)(zero_row + 1) * (K + 16) + (size_t)(zero_row + 1) * (K / 32);
    const size_t lds = sh ? ((lds_h + 15) & ~(size_t)15) + (size_t)M * (K + 8) * 2 : lds_h;
    // the h buffer descriptors (staged h, per-group scale loads) take 32-bit sizes and offsets; otherwise h is read
    // through 64-bit pointers
    const bool h32 = (long long)zero_row * ldh + K <= 0xFFFFFFFFll && (long long)zero_row * ldhs + K / 32 <= 0xFFFFFFFFll;
    // staged h: at most 60 KiB, which also bounds the per-thread load registers (DS_HV vectors, DS_HS bytes)
    const bool h_lds = h32 && lds <= 60 * 1024 && (long long)(zero_row + 1) * (K / 16) <= DS_HV * DS_WAVES * 64 &&
                       (long long)(zero_row + 1) * (K / 32) <= DS_HS * DS_WAVES * 64;
    const dim3 grid(N / 16), block(DS_WAVES * 64);
    // weight scales through LDS when every wave holds at most DS_SCG groups of <= 16 k-chunks and the scale rows are
    // 16-byte aligned for the wide loads
    const bool scl = h_lds && (n_slots + DS_WAVES - 1) / DS_WAVES <= DS_SCG && K / 128 <= 16 && (((uintptr_t)S) & 15) == 0 &&
                     (stride_se & 15) == 0;
    // h rows from global: per-group scale loads when a group's scales fit the wave's LDS region (<= 16 k-chunks), the
    // h scale rows hold >= 16 bytes and every wide load is aligned (16 bytes for the weight scales, 4 for h's)
    const bool gs = !h_lds && h32 && K / 128 <= 16 && K >= 512 && (((uintptr_t)S) & 15) == 0 && (stride_se & 15) == 0 &&
                    (ldhs & 3) == 0 && (((uintptr_t)hs) & 3) == 0;
    // the fused shared expert runs with the h rows staged in LDS only, through fewer staging registers
    if (sh && !(h_lds && (sh_fp8 || K / 32 <= DS_SHC * DS_WAVES) && (long long)(zero_row + 1) * (K / 16) <= DS_HV_SH * DS_WAVES * 64 &&
                (long long)(zero_row + 1) * (K / 32) <= DS_HS_SH * DS_WAVES * 64))
        return DSV41_EINVAL;
#define DS_LAUNCH(T, PF, NK, HL, SC) moe_down_sum_kernel<T, PF, NK, HL, SC><<<grid, block, HL ? lds : 0, st>>>(a)
#define DS_LAUNCH_SH(T, SC, SHV) moe_down_sum_kernel<T, DS_PF_SH, 0, 1, SC, SHV><<<grid, block, lds, st>>>(a)
    if (sh_fp8) {
        if (scl) { if (tiled) DS_LAUNCH_SH(1, 1, 2); else DS_LAUNCH_SH(0, 1, 2); }
        else { if (tiled) DS_LAUNCH_SH(1, 0, 2); else DS_LAUNCH_SH(0, 0, 2); }
        return (int)hipGetLastError();
    }
    if (sh) {
        if (scl) { if (tiled) DS_LAUNCH_SH(1, 1, 1); else DS_LAUNCH_SH(0, 1, 1); }
        else { if (tiled) DS_LAUNCH_SH(1, 0, 1); else DS_LAUNCH_SH(0, 0, 1); }
        return (int)hipGetLastError();
    }
#undef DS_LAUNCH_SH
    // weight tiles in flight per wave, measured at configs[1] (one token, 8 groups): 4 -> down launch 11.5 us, 12 -> 12.0,
    // 2 -> 12.2; and per layer 30.9 us with 4 against 31.0 / 31.05 / 31.2 us with 3 / 5 / 6; M = 4 (h rows in LDS, 32
    // groups) keeps 12 (4 in flight: 103.1 against 101.3 us per layer)
    if (scl) { if (tiled) DS_LAUNCH(1, 4, 0, 1, 1); else DS_LAUNCH(0, 4, 0, 1, 1); }
    else if (h_lds) { if (tiled) DS_LAUNCH(1, 12, 0, 1, 0); else DS_LAUNCH(0, 12, 0, 1, 0); }
    else if (gs) { if (tiled) DS_LAUNCH(1, 6, 0, 0, 2); else DS_LAUNCH(0, 6, 0, 0, 2); }
    else { if (tiled) DS_LAUNCH(1, 8, 0, 0, 0); else DS_LAUNCH(0, 8, 0, 0, 0); }
#undef DS_LAUNCH
    return (int)hipGetLastError();
}

// The down projection for M tokens through the run-split kernel and the fixed-order reduction (two launches); part:
// fp32 workspace of at least S * M * N floats, S = ceil(n_slots / Q) (at least 1), Q = max(1, min(32 - M,
// ceil(n_slots / 8))).
extern "C" int dsv41_moe_down_sum_split(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                                        int N, int K, const uint8_t* hc, long long ldh, const uint8_t* hs, long long ldhs,
                                        const int* grp_expert, const int* grp_start, const int* tok_sorted, int n_slots, int M,
                                        float* y, long long ldy, const uint16_t* ys, long long ldys, uint16_t* yb, long long ldyb,
                                        int shard_start, int shard_n, uint16_t* hres, const float* hpost, const float* hcomb,
                                        float* part, long long part_floats, void* stream) {
    if (!W || !S || !hc || !hs || !grp_expert || !grp_start || !tok_sorted || !part || (!y && !yb && !hres)) return DSV41_EINVAL;
    if (hres && (!hpost || !hcomb || (((uintptr_t)hres) & 7))) return DSV41_EINVAL;
    if (N <= 0 || (N & 127) || K < 128 || K > 2048 || (K & 127) || n_slots < 0 || n_slots > DS_MAX_SLOTS || M < 1 || M > 16)
        return DSV41_EINVAL;
    if (stride_we <= 0 || stride_we > 0xFFFFFFFFll || stride_se <= 0 || stride_se > 0xFFFFFFFFll || stride_we < (long long)N * (K / 2) ||
        stride_se < (long long)N * (K / 32))
        return DSV41_EINVAL;
    // the weight scales take 16-byte loads (tiled) or 4-byte loads (row-major); h rows 16-byte vectors, 32-bit offsets
    if ((((uintptr_t)S) & 15) || (stride_se & 15) || (ldh & 15) || (((uintptr_t)hc) & 15) || ldh < K || ldhs < K / 32 ||
        (long long)n_slots * ldh + K > 0xFFFFFFFFll || (long long)n_slots * ldhs + K / 32 > 0xFFFFFFFFll)
        return DSV41_EINVAL;
    if ((y && (ldy < N || (ldy & 3) || (((uintptr_t)y) & 15))) || (yb && ldyb < N) || (yb && ys && ldys < N) || (((uintptr_t)part) & 15))
        return DSV41_EINVAL;
    // runs of Q pair rows: at least 8 runs (so the grid fills the CUs), at most 32 - M rows each (the LDS rows)
    const int Q = max(1, min(32 - M, (n_slots + 7) / 8)), runs = n_slots > 0 ? (n_slots + Q - 1) / Q : 1;
    if (runs > DX_RUNS) return DSV41_EINVAL;
    if (part_floats < (long long)runs * M * N) return DSV41_EINVAL;
    DownSumArgs a{W, stride_we, S, stride_se, N, K, hc, ldh, hs, ldhs, n_slots, grp_expert, grp_start, tok_sorted, n_slots, M,
                  y, ldy, ys, ldys, yb, ldyb, shard_start, shard_n, nullptr, 0, nullptr, 0, 0.f, nullptr, 0, 0,
                  hres, hpost, hcomb, nullptr, 0};
    hipStream_t st = (hipStream_t)stream;
    const size_t lds = (size_t)DX_ROWS * (K + 16) + (size_t)DX_ROWS * (K / 32);
    const dim3 grid(N / 128, runs), block(DS_WAVES * 64);
#define DX_LAUNCH(T)                                                                                                  \
    do {                                                                                                          \
        const hipError_t err = hipFuncSetAttribute((const void*)moe_down_split_kernel<T, 8>,                     \
                                                   hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);         \
        if (err != hipSuccess) return (int)err;                                                                   \
        moe_down_split_kernel<T, 8><<<grid, block, lds, st>>>(a, part, Q);                                        \
    } while (0)
    if (tiled) DX_LAUNCH(1); else DX_LAUNCH(0);
#undef DX_LAUNCH
    const int nthr = M * (N / 4);
    down_reduce_kernel<<<(nthr + 255) / 256, 256, 0, st>>>(a, part, runs);
    return (int)hipGetLastError();
}
