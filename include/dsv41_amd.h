/* C ABI of libdsv41_amd.so: the MI355X (gfx950) FP4 MoE expert path.
 *
 * Every entry point takes raw device pointers, sizes, and the HIP stream to launch on (hipStream_t passed as
 * void*), launches its kernels on that stream and returns immediately (stream-ordered, capturable in a
 * hipGraph). Return value: 0 ok, -1 invalid arguments (nothing launched), -2 (dsv41_moe_experts_noalloc only) the
 * call needs more than the library's scratch array (nothing launched), > 0 the hipError_t of the launch.
 * No entry point allocates device memory; callers own every buffer.
 *
 * Formats (reference dsv41/quant.py:6-110):
 *   FP4 weights  uint8 [E][N][K/2], E2M1 nibbles, low nibble = even k; scales uint8 [E][N][K/32] E8M0 (2^(b-127)).
 *   tiled = 1: weights/scales in the reference's tile_fp4 / tile_fp4_scales layout (quant.py:113-139):
 *                [E][N/16][K/128][16 rows][64 B] and [E][N/16][K/128][16][4]; tiled = 0: row-major as above.
 *   FP8 activations: E4M3 (float8_e4m3fn) codes uint8 [rows][K] + E8M0 bytes uint8 [rows][K/32].
 *   bf16 tensors are passed as uint16_t bit patterns.
 */
#ifndef DSV41_AMD_H
#define DSV41_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 [rows][K] = E2M1 x 2^(S-127), bit-exact with quant.dequant_fp4 (quant.py:98-110). */
int dsv41_dequant_fp4(const uint8_t* w, const uint8_t* s, long long rows, int K, int tiled, uint16_t* out, void* stream);

/* Per-32 FP8 quantisation of bf16 (x_f32 = 0) or fp32 rows: E4M3 codes + E8M0 scales in natural k order, and/or
 * the fake-quantised values in the input dtype (fq). Replaces quant.fake_quant_fp8 / quant.quant_fp8
 * (quant.py:45-64) and fused.fake_quant_fp8 (fused.py:82-83). permuted = 1: x is in cukern.permute_x order
 * (cukern.py:221-227). Any of codes / scales / fq may be NULL (not all). */
int dsv41_quant_fp8(const void* x, int x_f32, long long rows, int K, long long ldx, int permuted,
                    uint8_t* codes, uint8_t* scales, void* fq, void* stream);

/* bf16 activations as two FP8 terms, so the FP4 GEMMs below honour the reference's bf16-operand contract (fp4_gemv.cu,
 * fp4_tcw.cu and moe_kernels.py:154-200 multiply bf16 x by bf16-decoded weights; cukern.py:60-77, 238-276 and
 * moe_kernels.py:127-151 accept any bf16 x): x = hi + lo per 32-group, hi = the codes and scales dsv41_quant_fp8 gives
 * (bit-identical), lo = the residual x - hi rounded to E4M3 with an E8M0 scale of its own. hi + lo == x for every
 * element whose residual is in the lo term's normal range; otherwise |x - hi - lo| < 2^-21 of the group's amax.
 * x: bf16 [rows][ldx] (ldx % 8 == 0, 16-byte aligned), 8-k permuted when permuted = 1 (codes in natural order).
 * Outputs: hc / lc [rows][K], hs / ls [rows][K/32], lo_flag (device int) cleared, then set to 1 when any lo code is
 * non-zero (FP8-grid x leaves it 0). No counterpart in the reference, which has no FP8 activation operand. */
int dsv41_quant_fp8_split(const uint16_t* x, long long rows, int K, long long ldx, int permuted, uint8_t* hc, uint8_t* hs,
                          uint8_t* lc, uint8_t* ls, int* lo_flag, void* stream);

/* h = fq8(bf16(wt * silu(min(g, L)) * clamp(u, +-L))) per 32 (fused.swiglu_quant, fused.py:283-345).
 * gu: fp32 [rows][ld_gu] (gu_bf16 = 0) or bf16 (gu_bf16 = 1, as fused.py:294 accepts), gate columns [0, inter), up
 * [inter, 2 inter); ld_gu in elements. wt: fp32 [rows] or NULL. Outputs (any
 * may be NULL, not all): FP8 codes [rows][inter] + E8M0 [rows][inter/32]; bf16 values [rows][inter]
 * (8-k permuted when permute = 1, fused.py:303-305). */
int dsv41_swiglu_quant(const void* gu, int gu_bf16, long long ld_gu, const float* wt, int rows, int inter, float limit,
                       uint8_t* codes, uint8_t* scales, uint16_t* h_bf16, int permute, void* stream);

/* Grouped FP4 x FP8 GEMM on block-scaled MFMA: for each group g (expert grp_expert[g], pairs
 * grp_start[g] .. grp_start[g+1]-1) and pair p: out[out_row ? out_row[p] : p][0:N] (=, +=, atomic += for
 * accum 0 / 1 / 2) (pair_wt ? pair_wt[p] : 1) * sum_k x[pair_tok[p]][k] * deq(W[e])[n][k].
 * Replaces cukern.fp4_gemm_tc (cukern.py:238-276, fp4_tcw.cu / fp4_tc.cu), cukern.fp4_gemv_pairs
 * (cukern.py:60-77, fp4_gemv.cu) and moe_kernels.grouped_fp4_gemm (moe_kernels.py:127-200).
 * W / S hold the experts shard_start .. shard_start + shard_n - 1 (shard_n = the experts W holds when unsharded),
 * stride_we >= N * K / 2 and stride_se >= N * K / 32 bytes apart. Groups of any size (max_tokens selects the
 * pass width); groups whose expert is outside [shard_start, shard_start + shard_n) are skipped and, with
 * zero_out, their rows zeroed (cukern.py:244-246); padding groups (expert < 0) and groups with fewer than min_tok
 * or more than max_tok pairs are skipped. Bounds: group ranges are clamped to [0, n_pairs); pairs whose token is
 * outside [0, x_rows) contribute zeros; output rows outside [0, out_rows) are not written. N % 16 == 0,
 * K % 128 == 0. xlc / xls / lo_flag (all three or none): the lo term of dsv41_quant_fp8_split, with xc / xs its hi
 * term; x is then hi + lo, and the lo term's products are added only when *lo_flag is non-zero (FP8-grid input runs
 * the one-term arithmetic bit for bit). */
int dsv41_fp4_grouped_gemm(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                           int N, int K, const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, int x_rows,
                           const uint8_t* xlc, const uint8_t* xls, const int* lo_flag, const int* grp_expert, const int* grp_start, int G, const int* pair_tok, int n_pairs,
                           float* out, long long ldo, int out_rows, const int* out_row, const float* pair_wt, int accum,
                           int max_tokens, int shard_start, int shard_n, int zero_out, int min_tok, int max_tok, void* stream);

/* dsv41_fp4_grouped_gemm on bf16 activations x [x_rows][ldx] (ldx in elements, a multiple of 8; x 16-byte aligned;
 * 8-k permuted rows when permuted, as fp4_gemm_tc takes them, cukern.py:224-227): the kernel splits each staged row
 * into the two FP8 terms of dsv41_quant_fp8_split itself, so the reference's bf16-activation call
 * (cukern.fp4_gemm_tc / fp4_gemv_pairs, cukern.py:60-77, 238-276) runs as one launch. Only where both terms of
 * min(max_tokens, 8) rows fit the kernel's 48 KiB of LDS staging, 2 (min(max_tokens, 8) (K + 16 + K / 32)) bytes
 * rounded up to 16: otherwise -1 (the caller quantises with dsv41_quant_fp8_split and calls
 * dsv41_fp4_grouped_gemm). */
int dsv41_fp4_grouped_gemm_bf16(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                                int N, int K, const uint16_t* x, long long ldx, int x_rows, int permuted,
                                const int* grp_expert, const int* grp_start, int G, const int* pair_tok, int n_pairs,
                                float* out, long long ldo, int out_rows, const int* out_row, const float* pair_wt, int accum,
                                int max_tokens, int shard_start, int shard_n, int zero_out, int min_tok, int max_tok, void* stream);

/* Decode routing + up projection + SwiGLU in one launch (M <= 16 tokens, topk <= 16, E <= 512):
 * routing from fp32 logits [M][ldl] (gate_topk semantics, score_func 0 sqrt(softplus) / 1 sigmoid / 2 softmax;
 * bias may be NULL; the logits may be nparts partial sums part_stride floats apart, added in ascending order) or, with logits = NULL, from given eid_in / wt_in [M][topk]; the (token, expert) pairs are
 * bucketed by expert (groups in ascending expert id, tokens ascending inside a group); x bf16 [M][ldx] on the
 * FP8 grid is quantised to E4M3 + E8M0 in LDS, and h = fq8(bf16(wt * silu(min(g, L)) * clamp(u, +-L))) of
 * gu = x . deq(W13[e])^T (2 * I rows: w1 then w3) is written as FP8 codes hc [P][ldhc] + E8M0 hs [P][ldhs],
 * P = M * topk pair slots in sorted order. Outputs for dsv41_moe_down_sum: grp_expert [P] (-1 past the last
 * group), grp_start [P + 1], tok_sorted [P], wt_sorted [P]; routing eid_out / wt_out [M][topk] (optional).
 * Expert ids outside [0, E) are dropped. Replaces gate_topk + moe_dispatch + the w13 fp4_gemm_tc + swiglu_quant
 * of decode.DecodeRuntime.moe2 / experts_tc (decode.py:354-361, 316-335; fused2.py:418-452; cukern.py:238-276;
 * fused.py:283-345; p2p.cu:90-132).
 * Optional bf16 shared expert (Ws13 = [w1; w3] bf16 [2I][ldws], or NULL; sh_tiled = 1: in 16 x 32 tiles of 1 KiB,
 * [2I/16][H/32][16][32] with ldws = H): the same launch also writes its gate/up gus = bf16(x . Ws13^T) as bf16
 * [M][ldgus] (linear_w(xq, sh_w13), decode.py:368), for dsv41_moe_down_sum. With Ss13 non-NULL the shared expert is FP8
 * (w8.W8, w8.py:57-124): Ws13 points at E4M3 bytes in the w8 tile order [2I/16][H/64][4][16][16 B] (sh_tiled = 1,
 * ldws = H bytes) and Ss13 at its E8M0 block scales [2I/32][ldss13]; gus is the same bf16 gate/up. */
int dsv41_moe_decode_up(const float* logits, long long ldl, int nparts, long long part_stride, const float* bias, float temp,
                        float route_scale, int score_func, int norm, const int* eid_in, const float* wt_in, int M, int topk, int E, const uint16_t* x,
                        long long ldx, const uint8_t* W13, long long stride_we, const uint8_t* S13, long long stride_se,
                        int tiled, int H, int I, float limit, uint8_t* hc, long long ldhc, uint8_t* hs, long long ldhs,
                        int* eid_out, float* wt_out, int* grp_expert, int* grp_start, int* tok_sorted, float* wt_sorted,
                        const uint16_t* Ws13, long long ldws, int sh_tiled, uint16_t* gus, long long ldgus, const uint8_t* Ss13,
                        long long ldss13, void* stream);

/* The same launch with the M tokens taken pair by pair (same arguments and outputs; for M = 1 identical to
 * dsv41_moe_decode_up). Grid row g is pair g = (token g / topk, pick g % topk): its workgroups route that token
 * themselves (one wave runs the token's gate and posts pick g % topk as soon as its round is done, the token's row is
 * staged meanwhile) and stream that pick's expert; h of pair g goes to row g. The tables describe P groups of one pair
 * each: grp_expert[g] = the pair's expert (-1 for an id outside [0, E)), grp_start[g] = g, tok_sorted[g] = g / topk,
 * wt_sorted[g] = its weight, grp_start[P] = P. No separate gate launch and no bucketing; an expert that several tokens
 * picked is read once per pair. Replaces the same reference steps as dsv41_moe_decode_up (decode.py:354-361,
 * 316-335). H / 16 <= 448. */
int dsv41_moe_decode_up_pairs(const float* logits, long long ldl, int nparts, long long part_stride, const float* bias, float temp,
                              float route_scale, int score_func, int norm, const int* eid_in, const float* wt_in, int M, int topk, int E,
                              const uint16_t* x, long long ldx, const uint8_t* W13, long long stride_we, const uint8_t* S13,
                              long long stride_se, int tiled, int H, int I, float limit, uint8_t* hc, long long ldhc, uint8_t* hs,
                              long long ldhs, int* eid_out, float* wt_out, int* grp_expert, int* grp_start, int* tok_sorted,
                              float* wt_sorted, const uint16_t* Ws13, long long ldws, int sh_tiled, uint16_t* gus, long long ldgus,
                              const uint8_t* Ss13, long long ldss13, void* stream);

/* Decode down projection and per-token combine: y[t][n] = sum over groups g and their pair p of token t of
 * h_p . deq(W2[e_g])[n]  (M <= 16 tokens, n_slots <= 256 group slots; slots with expert -1 are unused).
 * zero_row: index of an all-zero row of hc and hs (read for tokens a group does not contain).
 * Optional outputs: y fp32 [M][ldy]; yb bf16 = bf16(y + ys) with ys the bf16 shared-expert output or NULL.
 * Replaces the w2 call of decode.DecodeRuntime.experts_tc (decode.py:316-335) plus the sum of the k rows in
 * fused2.hc_post2_ (fused2.py:490-495) and model.MoE.__call__ (model.py:581, 590-591).
 * Optional bf16 shared expert in the same launch (Ws2 bf16 [N][ldws2], or NULL; then ys must be NULL; sh_tiled = 1:
 * Ws2 in 16 x 32 tiles of 1 KiB, [N/16][K/32][16][32] with ldws2 = K): from gus
 * (dsv41_moe_decode_up's bf16 gate/up [M][ldgus]) each workgroup forms h_s = swiglu_quant(gus, no weight, limit)
 * (model.py:410) and adds ys = bf16(h_s . Ws2^T) (linear_w(hs, sh_w2), decode.py:370) to y before the bf16 rounding
 * of yb; ys_out (bf16 [M][ldyso], optional) receives ys. Needs the h rows and h_s in 60 KiB of LDS
 * ((n_slots + 1)(K + 16 + K / 32) + 2 M (K + 8) bytes, e.g. M <= 2 at K = 1664) and M K <= 4096; else -1.
 * Optional hyper-connection post mix in the same epilogue (hres bf16 residual, token t's 4 streams at hres + 4 N t + N i;
 * hpost fp32 [M][4]; hcomb fp32 [M][4][4]; or NULL): r_i <- bf16(post[t][i] x + sum_j comb[t][j][i] r_j) with
 * x = bf16(y + ys), in place (fused2.hc_post2_, fused2.py:476-508), replacing its separate launch.
 * With Ss2 non-NULL the shared expert is FP8: Ws2 points at E4M3 bytes in the w8 tile order [N/16][K/64][4][16][16 B]
 * (sh_tiled = 1, ldws2 = K bytes, K / 64 <= 40) and Ss2 at its E8M0 block scales [N/32][ldss2]. */
int dsv41_moe_down_sum(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled,
                       int N, int K, const uint8_t* hc, long long ldh, const uint8_t* hs, long long ldhs, int zero_row,
                       const int* grp_expert, const int* grp_start, const int* tok_sorted, int n_slots, int M,
                       float* y, long long ldy, const uint16_t* ys, long long ldys, uint16_t* yb, long long ldyb,
                       int shard_start, int shard_n, const uint16_t* gus, long long ldgus, const uint16_t* Ws2,
                       long long ldws2, int sh_tiled, float limit, uint16_t* ys_out, long long ldyso, uint16_t* hres,
                       const float* hpost, const float* hcomb, const uint8_t* Ss2,
                       long long ldss2, void* stream);

/* The down projection of dsv41_moe_down_sum (no fused shared expert) for M tokens whose h rows do not fit LDS at
 * once: the groups are split into runs of Q = max(1, min(32 - M, ceil(n_slots / 8))) consecutive pair rows, each
 * workgroup computes 128 output rows over one run with that run's h rows in LDS, and a second launch adds the runs'
 * fp32 partial sums in run order before the epilogue (y, bf16(y + ys), the hyper-connection post mix). part: fp32
 * workspace of at least S * M * N floats, S = ceil(n_slots / Q) (>= 1). N % 128 == 0, K % 128 == 0, K <= 2048.
 * Replaces the same calls as
 * dsv41_moe_down_sum (decode.py:324-335). */
int dsv41_moe_down_sum_split(const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled, int N, int K,
                             const uint8_t* hc, long long ldh, const uint8_t* hs, long long ldhs, const int* grp_expert,
                             const int* grp_start, const int* tok_sorted, int n_slots, int M, float* y, long long ldy,
                             const uint16_t* ys, long long ldys, uint16_t* yb, long long ldyb, int shard_start, int shard_n,
                             uint16_t* hres, const float* hpost, const float* hcomb, float* part, long long part_floats,
                             void* stream);

/* Prefill w13 + SwiGLU: for every group g of <= 256 expert-sorted pairs (moe_dispatch tables with gmax <= 256;
 * groups of more than 128 pairs run on a 256-pair tile),
 * h[p] = fq8(bf16(wt_sorted[p] * silu(min(g, L)) * clamp(u, +-L))) with gu = x[tok_sorted[p]] . deq(W13[e])^T;
 * x as E4M3 codes xc [x_rows][ldx] + E8M0 xs [x_rows][ldxs] (x_rows * ldx < 2^32); h as FP8 codes hc [P][ldhc]
 * + E8M0 hs [P][ldhs] in sorted pair order. H % 128 == 0, H >= 384, I % 64 == 0. Replaces the w13 grouped_fp4_gemm + swiglu_quant of
 * model.MoE.__call__ (model.py:584-587; moe_kernels.py:127-151; fused.py:283-345). grp_order (optional, [G]): the order
 * the launch takes the groups in (dsv41_group_order: largest first); NULL: table order. The result is the same either way. */
int dsv41_prefill_up(const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, int x_rows, const uint8_t* W13, long long stride_we,
                     const uint8_t* S13, long long stride_se, int tiled, int E, int H, int I, const int* grp_expert,
                     const int* grp_start, int G, const int* tok_sorted, const float* wt_sorted, float limit, uint8_t* hc,
                     long long ldhc, uint8_t* hs, long long ldhs, const int* grp_order, void* stream);

/* Prefill w2: y2[p] = h[p] . deq(W2[e_g])^T (fp32 [P][ldy], sorted pair order) for the same groups; h_rows = P
 * (h_rows * ldhc < 2^32).
 * I % 128 == 0, I >= 384, H % 128 == 0. Replaces the w2 grouped_fp4_gemm of model.py:588. grp_order: as in dsv41_prefill_up. */
int dsv41_prefill_down(const uint8_t* hc, long long ldhc, const uint8_t* hs, long long ldhs, int h_rows, const uint8_t* W2, long long stride_we,
                       const uint8_t* S2, long long stride_se, int tiled, int E, int H, int I, const int* grp_expert,
                       const int* grp_start, int G, float* y2, long long ldy, const int* grp_order, void* stream);

/* The groups 0 .. G-1 of a dispatch (moe_dispatch tables) ordered by pair count, largest first, into order [G] (a
 * permutation; within one count the order is unspecified). Groups whose expert is -1 count 0; pair ranges are clamped to
 * [0, n_pairs) and counts to 256. No counterpart in the reference: it lets the prefill launches start their longest items
 * first, so none of them starts near the end of a launch (scheduling only, the results do not change). */
int dsv41_group_order(const int* grp_expert, const int* grp_start, int G, int n_pairs, int* order, void* stream);

/* The w2 kernel of the prefill path as a general grouped GEMM for groups of up to 128 pairs (the 256-row x 128-pair tile
 * kernel): for each group g (expert grp_expert[g] in [0, E), pairs grp_start[g] .. grp_start[g+1]-1, clamped to
 * [0, n_pairs), at most the first 128 of a group are computed) and pair p: y[p][0:N] = x[row][:] . deq(W[e])^T with
 * row = row_of_pair ? row_of_pair[p] : p (rows outside [0, x_rows) read zeros). x: E4M3 codes [x_rows][ldx] + E8M0
 * [x_rows][ldxs]. Rows of y for pairs outside every computed group are not written. N % 256 == 0, K % 128 == 0,
 * K >= 384. Serves moe_kernels.grouped_fp4_gemm (moe_kernels.py:127-200) and cukern.fp4_gemm_tc (cukern.py:238-276)
 * when their groups exceed 16 pairs: the weights of a group are read once for up to 128 pairs. xlc / xls / lo_flag
 * (all or none): the lo term of dsv41_quant_fp8_split, added by a second pass over the groups that does nothing when
 * *lo_flag is 0. */
int dsv41_fp4_grouped_gemm_t128(const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, int x_rows,
                                const uint8_t* xlc, const uint8_t* xls, const int* lo_flag, const int* row_of_pair,
                                const uint8_t* W, long long stride_we, const uint8_t* S, long long stride_se, int tiled, int E, int N,
                                int K, const int* grp_expert, const int* grp_start, int G, int n_pairs, float* y, long long ldy,
                                void* stream);

/* moe_kernels.grouped_fp4_gemm with the reference kernel's own epilogue (moe_kernels.py:29-80, 155-200: the tile scaled
 * by the pair weights, then tl.atomic_add into the output rows), on the prefill tile kernels for groups of up to 256
 * pairs (128-pair tiles, 256-pair tiles for groups of more than 128): for each group g (expert in [0, E), pairs clamped
 * to [0, n_pairs), at most the first 256 computed) and pair p: out[row_out[p]][0:N] += fl(wt[p] * (x[row] .
 * deq(W[e])^T)), row as in dsv41_fp4_grouped_gemm_t128; output rows outside [0, out_rows) are skipped. distinct: a
 * device int (or NULL) that is non-zero when no two pairs share an output row; then accum == 0 stores (out must hold
 * zeros beforehand) and accum == 1 reads, adds and writes, deterministically; otherwise fp32 atomic adds (any order,
 * as the reference's). y2: workspace fp32 [n_pairs][ldy2] (the unweighted pair rows, sorted order). G <= 65535.
 * N % 256 == 0, K % 128 == 0, K >= 384, ldo % 4 == 0 and ldy2 % 4 == 0, out and y2 16-byte aligned. xlc / xls /
 * lo_flag: the lo term, as for dsv41_fp4_grouped_gemm_t128 (its pass adds into y2 before the scatter). */
int dsv41_fp4_grouped_gemm_scatter(const uint8_t* xc, long long ldx, const uint8_t* xs, long long ldxs, int x_rows,
                                   const uint8_t* xlc, const uint8_t* xls, const int* lo_flag, const int* row_of_pair, const uint8_t* W, long long stride_we, const uint8_t* S,
                                   long long stride_se, int tiled, int E, int N, int K, const int* grp_expert, const int* grp_start,
                                   int G, int n_pairs, const int* row_out, const float* wt, const int* distinct, int accum,
                                   float* out, long long ldo, int out_rows, float* y2, long long ldy2, void* stream);

/* The distinct-rows flag of dsv41_fp4_grouped_gemm_scatter (no counterpart in the reference, whose kernel always adds
 * atomically): *flag (device int) = 1 when no two of the first n_placed entries of row_out (n_placed: a device int,
 * e.g. the dispatch's placed-pair count grp_start[n]; NULL: n) that lie in [0, out_rows) are equal, else 0; 0 without
 * checking when out_rows > 2^20. One workgroup, no host round trip. */
int dsv41_rows_distinct(const int* row_out, int n, const int* n_placed, int out_rows, int* flag, void* stream);

/* Combine: y[t] = sum_j y2[inv[t * topk + j]] for j ascending (model.py:589, view(n, k, dim).sum(1)), fp32 into
 * y32 and/or bf16(y + ys) into out (model.py:590-591; ys NULL: no shared expert). inv: moe_dispatch's inverse
 * permutation; an entry of -1 (a dropped pair) contributes nothing. N % 4 == 0. */
int dsv41_combine_pairs(const float* y2, long long ldy2, const int* inv, int topk, int T, int N, const uint16_t* ys, long long ldys,
                        uint16_t* out, long long ldo, float* y32, long long ld32, void* stream);

/* out[t][n] = sum_k x[t][k] * W[n][k], bf16 W [N][ldw] (tiled = 1: 16 x 32 tiles of 1 KiB, [N/16][K/32][16][32] with
 * ldw = K), bf16 x [M][ldx], M <= 16, fp32 and/or bf16 output.
 * The bf16 shared expert's two GEMVs (model.MoE.shared_expert, model.py:409-412; decode.py:369-371) and the
 * router logits (decode.py:357, model.py:391-392). */
int dsv41_dense_gemv_bf16(const uint16_t* W, long long ldw, int tiled, int N, int K, const uint16_t* x, long long ldx, int M,
                          float* out, long long ldo, uint16_t* outb, long long ldob, void* stream);

/* Layer-to-layer step of the decode stack, per token row (M rows, H <= 8192, H % 32 == 0): r = bf16(x + y),
 * xn = bf16(r * rsqrt(mean(r^2) + eps) * w) (fused.rmsnorm, fused.py:92-110; w NULL = ones) and
 * xq = fake_quant_fp8(xn) (quant.py:34-54), all bf16. xn feeds the next router (model.py:391-392 routes on the
 * unquantised activations), xq the next experts. No reference entry point: it stands in for the attention
 * block between two MoE layers when the expert path runs as a stack. */
int dsv41_residual_rmsnorm_quant(const uint16_t* x, long long ldx, const uint16_t* y, long long ldy, const uint16_t* w, float eps,
                                 int M, int H, uint16_t* xn, long long ldn, uint16_t* xq, long long ldq, void* stream);

/* Router logits of the next layer with the layer-to-layer step fused in (M <= 16 rows, H % 1024 == 0, E % 16 == 0):
 * r = bf16(x + y) (y NULL: r = x), xn = bf16(r * rsqrt(mean(r^2) + eps) * w) (fused.rmsnorm, fused.py:92-110;
 * w NULL = ones), logits = xn . G^T (bf16 G [E][ldg]; model.py:391-392, decode.py:357) written as KS = H / 1024
 * partial sums part [KS][M][E] for dsv41_gate_topk / dsv41_moe_decode_up (nparts = KS, part_stride = M * E).
 * Also writes xn and xq = fake_quant_fp8(xn) (quant.py:34-54), bf16 [M][H]. */
int dsv41_router_logits(const uint16_t* x, long long ldx, const uint16_t* y, long long ldy, const uint16_t* w, float eps,
                        const uint16_t* G, long long ldg, int E, int H, int M, float* part, uint16_t* xn, long long ldn,
                        uint16_t* xq, long long ldq, void* stream);

/* Router logits with fp32 router weights (model.MoE.gate: F.linear(x.float(), gate_w), gate_w fp32 [E][ldg],
 * model.py:368, 392) for M <= 16 bf16 rows x [M][ldx]: KS = H / 1024 partial sums part [KS][M][E] (k ranges of 1024,
 * ascending), which dsv41_gate_topk / dsv41_moe_decode_up add in part order (nparts = KS, part_stride = M * E).
 * H % 1024 == 0. */
int dsv41_router_logits_f32w(const uint16_t* x, long long ldx, const float* G, long long ldg, int E, int H, int M, float* part,
                             void* stream);

/* The decode block's hyper-connection steps either side of the experts (hc <= 4 residual streams):
 * pre (fused2.hc_pre_norm_quant2, fused2.py:189-236): per row b, a = bf16(sum_h pre[b][h] * x[b][h]) (x bf16 [B][ldx], the
 * hc streams D apart; pre fp32 [B][ldp]), y = bf16(a * (1 / sqrt(mean(a^2) + eps)) * w) (w bf16 [D]), yq =
 * fake_quant_fp8(y); optional yf = y as fp32 and yqp = yq in the 8-k permuted order (fused2.py:113-117). D % 32 == 0. */
int dsv41_hc_pre_norm_quant(const uint16_t* x, long long ldx, int hc, const float* pre, long long ldp, const uint16_t* w, float eps,
                            int B, int D, uint16_t* y, long long ldy, uint16_t* yq, long long ldq, float* yf, long long ldf,
                            uint16_t* yqp, long long ldqp, void* stream);

/* post (fused2.hc_post2_, fused2.py:474-538), in place on the residual res bf16 [B][ldr] (4 streams D apart): per row b
 * and column n, x = bf16(sum_{k < nsum} y2[b][k][n] + ys[b][n]) (y2 fp32 at y2 + b y2_row + k y2_sum; ys bf16 or NULL),
 * or the given bf16 x when nsum = 0; then r[i] <- bf16(post[b][i] x + sum_j comb[b][j][i] r[j]) (post fp32 [B][ldpost],
 * comb fp32 [B][ldcomb] as 4 x 4 row-major). D % 4 == 0. */
int dsv41_hc_post(const uint16_t* x, long long ldx, const float* y2, long long y2_row, long long y2_sum, int nsum, const uint16_t* ys,
                  long long ldys, uint16_t* res, long long ldr, const float* post, long long ldpost, const float* comb, long long ldcomb,
                  int B, int D, void* stream);

/* Dense FP8 weights x bf16 activations, M <= 64 output rows (cukern.fp8_gemm_tc, cukern.py:98-173, and
 * cukern.fp8_gemv, cukern.py:78-93, behind w8.linear_w / w8.oproj_a, w8.py:102-124):
 * out[t][n] = sum_k x[t'][k] * e4m3(W[n][k]) * 2^(S[n / 32][k / 32] - 127), fp32 accumulation, fp32 and/or bf16 output.
 * W: E4M3 bytes, natural row-major [N][ldw] or (tiled = 1) [N/16][K/64][4][16][16 B] with ldw = K (N % 16 == 0);
 * S: E8M0 bytes [ceil(N/32)][lds]. x bf16 rows ldx apart; t' = t, or with group_cols > 0 (block-diagonal use,
 * w8.oproj_a) t' = t * (N / group_cols) + n / group_cols (group_cols % 16 == 0). K % 64 == 0. Deterministic; no workspace. */
int dsv41_fp8_gemm(const uint8_t* W, long long ldw, int tiled, const uint8_t* S, long long lds, int N, int K,
                   const uint16_t* x, long long ldx, int M, int group_cols, float* out, long long ldo,
                   uint16_t* outb, long long ldob, void* stream);

/* W8.bf16 / quant.dequant_fp8_block (w8.py:78-82, quant.py:90-95): out bf16 [N][ldo] = bf16(e4m3(W) * 2^(S - 127)),
 * the fp32 product rounded to bf16 (bit-exact). W in either layout of dsv41_fp8_gemm (tiled needs K % 64 == 0);
 * K % 16 == 0. */
int dsv41_dequant_fp8(const uint8_t* W, long long ldw, int tiled, const uint8_t* S, long long lds, int N, int K,
                      uint16_t* out, long long ldo, void* stream);

/* MoE gate on logits: score_func 0 sqrt(softplus), 1 sigmoid, 2 softmax; top-k of scores + bias (lowest index
 * wins ties); weights renormalised when norm, times route_scale. fused2.gate_topk (fused2.py:418-471),
 * model.MoE.gate (model.py:391-404). nparts > 1: scores are that many partial sums part_stride floats apart
 * (dsv41_router_logits output), added in ascending order; nparts = 1: plain scores. */
int dsv41_gate_topk(const float* scores, long long lds, const float* bias, int B, int E, float temp, int topk, float route_scale,
                    int score_func, int norm, int* eid, float* wt, int nparts, long long part_stride, void* stream);

/* Expert bucketing of n = tokens * topk pairs: tok_sorted, wt_sorted, inv, grp_expert (-1 padded), grp_start
 * (padded with the number of placed pairs, n when every id is valid), groups of <= gmax pairs per expert;
 * n_groups (optional) receives the group count. Pairs keep ascending order within an expert. Ids outside [0, E)
 * are dropped: their inv entry is -1 and the sorted slots past the placed pairs hold token 0, weight 0.
 * cukern.moe_dispatch (cukern.py:323-337, p2p.cu:90-132); E <= 512. */
int dsv41_moe_dispatch(const int* eid, const float* wt, int n, int topk, int E, int gmax, int* tok_sorted, float* wt_sorted,
                       int* inv, int* grp_expert, int* grp_start, int* n_groups, void* stream);

/* Decode routed experts without allocating (no counterpart in the reference): the same computation and the same
 * results as dsv41_moe_decode_up followed by dsv41_moe_down_sum (arguments as there; the W13 / W2 expert strides are
 * stride_w13 / stride_w2 and their scales' stride_s13 / stride_s2), for callers that cannot allocate device memory
 * (code under graph capture that must not call hipMalloc, serving loops, harnesses that forbid allocation). The h
 * rows and bucketing tables live in a 2 MiB device array of the library, one per GPU, held until the process
 * ends; nothing is allocated or freed. Returns -2 when a call needs more than that array: (M topk + 1) (I + I / 32)
 * bytes plus the tables, e.g. M = 16, topk = 8, I = 1664 needs 0.22 MiB. Calls on one GPU share the array: calls
 * that overlap in time on that GPU (other streams, other host threads) race. I % 128 == 0. */
int dsv41_moe_experts_noalloc(const float* logits, long long ldl, int nparts, long long part_stride, const float* bias, float temp,
                              float route_scale, int score_func, int norm, const int* eid_in, const float* wt_in, int M, int topk, int E,
                              const uint16_t* x, long long ldx, const uint8_t* W13, long long stride_w13, const uint8_t* S13,
                              long long stride_s13, const uint8_t* W2, long long stride_w2, const uint8_t* S2, long long stride_s2,
                              int tiled, int H, int I, float limit, int* eid_out, float* wt_out, float* y, long long ldy,
                              const uint16_t* ys, long long ldys, uint16_t* yb, long long ldyb, void* stream);

/* Diagnostics (no reference counterpart): one wave runs one matrix instruction on caller-given operands so a
 * test can check the lane layouts the kernels rely on. a, b: [64][8] dwords; sa, sb: [64]; c: [64][4] fp32. */
int dsv41_selftest_mfma_scale(const int* a, const int* b, const int* sa, const int* sb, float* c, int fmt_a, int fmt_b, void* stream);
int dsv41_selftest_mfma_bf16(const uint16_t* a, const uint16_t* b, float* c, void* stream);

/* Diagnostic: the matrix pipes' sustained rate for one operand mix (no counterpart in the reference): blocks x 256 threads
 * each run iters rounds of 8 independent v_mfma_scale_f32_16x16x128_f8f6f4 on registers. mode 0 FP4 x FP8, 1 FP8 x FP8,
 * 2 FP4 x FP4. FLOP per launch = blocks x 4 waves x iters x 8 x 2 x 16 x 16 x 128. out: one float, written only in a
 * case that does not occur (keeps the work live). */
int dsv41_selftest_mfma_rate(int mode, int blocks, int iters, float* out, void* stream);

/* Diagnostic: the HBM stream rate of a launch shape (no counterpart in the reference): blocks workgroups of `waves` (4 or 8)
 * waves read `tiles` 1 KiB tiles of src once with the decode kernels' nontemporal buffer loads, 8 tiles in flight per wave;
 * workgroup b reads the contiguous tiles [tiles b / blocks, tiles (b + 1) / blocks), its waves interleaved. sync = 1 adds a
 * workgroup barrier after every second tile (the prefill kernels' per-k-step synchronisation). out: one word, written only
 * if the bytes read XOR to one particular word (keeps the loads live). Bytes read per launch = 1024 tiles. */
int dsv41_selftest_stream(const uint8_t* src, long long tiles, int blocks, int waves, int sync, unsigned* out, void* stream);

/* FP8 conversion check (no counterpart in the reference: it validates this build's use of the gfx950 conversion
 * instructions against the bit-arithmetic rounding of quant.py:45-54): for each of the n inputs, the E4M3 code of
 * v[i] / 2^e[i] (clamped to +-448, round to nearest even) by bit arithmetic and by v_cvt_pk_fp8_f32 (both halves of a
 * pair), and the value of the first code decoded by bit arithmetic and by v_cvt_f32_fp8. out: [n][5] words. */
int dsv41_selftest_fp8_cvt(const float* v, const int* e, int n, uint32_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV41_AMD_H */
