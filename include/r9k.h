/* r9k.h -- C-ABI of libr9k.so, the gfx950 (MI355X) kernels of r9700-stack's quantized-MoE hot path.
 *
 * Drop-in for the symbols the reference's Python binds with ctypes (r9700_vllm/kernels/moe.py:22-57,
 * r9700_vllm/moe/route.py:40-52, r9700_vllm/kernels/moe.py:557-571): same names, same argument lists (pointers are
 * raw device addresses passed as `long`, sizes as `int`), same meaning, 0 on success and a negative (GEMMs, quant)
 * or nonzero (route, sum) code on a bad shape. Every call is ONE asynchronous launch group on `stream`
 * (a hipStream_t); nothing allocates, frees or synchronises, so calls are HIP-graph capturable. The caller owns
 * every buffer.
 *
 * Layouts that differ from the reference (the layout is the kernel's, produced by r9700_vllm/kernels/moe.py):
 *   wq  [E][N*K/2 bytes]: per 16-row column tile, 1 KB per 128-K tile = one 16x16x128 scaled-MFMA B operand
 *       (permute_fragments). Same size as the checkpoint codes, so weight prep stays in place.
 *   ws  [E][(K/32 + 1) * N bytes]: e8m0 exponents in the kernel's fragment order + the per-row max (pack_scales).
 * Knobs that only meant something on gfx1201 (WV, SK, NPW as the reference passes them, the LDS-A and fold bits of
 * MT, wref) are accepted and ignored; the routing-block contract is honoured: blk = 16 * (MT & 7) rows at decode,
 * r9k_moe_prefill_bm(cfg) rows in the prefill entry. r9k_moe_mxfp4a8 alone reads (WV, SK, NPW) as its gfx950 launch
 * shape, and only when the caller sets MT bit 5 (R9K_MT_SHAPE), which the reference never does.
 */
#ifndef R9K_H
#define R9K_H

#ifdef __cplusplus
extern "C" {
#endif

/* Grouped MXFP4 x fp8 GEMM, decode family. Replaces kernels/r9k_moe_mxfp4a8.hip:631-638 (r9k_moe_mxfp4a8).
 * out[r, n] = bf16((sum_k A[r / a_row_div, k] * W_e[n, k]) * (As[r / a_row_div] * topk_w[r])) for every routed
 * flat row r of the align tables (sorted_ids / expert_ids / ntpp, blocks of 16 * (MT & 7) rows).
 * a e4m3 [Ma][K]; as fp32 [Ma]; wq / ws as above (ws_estride = bytes per expert of ws); c bf16 [numel][N];
 * topk_w fp32 [numel] or 0. With MT & R9K_MT_SHAPE, (WV, SK, NPW) is the gfx950 launch shape -- K-tiles per load
 * batch, waves splitting K, 16-column tiles per wave, each 1, 2 or 4 (kernels/tuned.json via pick_cfg); without it
 * the kernel picks the shape and ignores them (the reference passes its gfx1201 knobs there). Errors: -1 N % 16,
 * -2 K % 32, -3 bad argument, -5 launch shape not built (R9K_MT_SHAPE set), -7 bad MT, -6 launch error. */
#define R9K_MT_SHAPE 32
int r9k_moe_mxfp4a8(long a, long as, long wq, long ws, long wref, long c, long sorted_ids, long expert_ids,
                    long ntpp, long topk_w, long ws_estride, long wref_estride, int max_blocks, int numel,
                    int a_row_div, int K, int N, int WV, int SK, int NPW, int MT, long stream);

/* Fused decode variants of the same GEMM. Replaces kernels/r9k_moe_mxfp4a8.hip:618-626 (r9k_moe_mxfp4a8_f).
 * fuse 1: gate_up with the activation in the epilogue: c fp32 [numel][N / 2] = silu(g) * u of the bf16-rounded gate
 * (columns n) and up (columns n + N / 2) outputs; N % 32 == 0. fuse 2: down with a = fp32 [numel][K] (fuse 1's
 * output) quantised per row on load (e4m3, scale absmax / 448, the r9k_silu_mul_quant_fp8 rule), as ignored (may be
 * 0), a_row_div 1. Routing blocks of 16 rows: MT & 7 must be 1 (-7). Results equal the unfused chain's bit for bit.
 * -8 fuse not 1 or 2; other errors as r9k_moe_mxfp4a8. */
int r9k_moe_mxfp4a8_f(int fuse, long a, long as, long wq, long ws, long wref, long c, long sorted_ids,
                      long expert_ids, long ntpp, long topk_w, long ws_estride, long wref_estride, int max_blocks,
                      int numel, int a_row_div, int K, int N, int WV, int SK, int NPW, int MT, long stream);

/* Prefill entry of the same GEMM. Replaces kernels/r9k_moe_mxfp4a8.hip:1227-1230 (r9k_moe_4bit_prefill).
 * nv: 0 MXFP4 (2, the reference's folded MXFP4, is the same data here); 1 native NVFP4 (ws / wref = the scales and
 * per-row fp32 multipliers of r9k_moe_nvfp4a8, wref_estride floats; cfgs with 128- or 256-row blocks, else -7);
 * 3 fp8 weights returns -8.
 * Tables built with blk = r9k_moe_prefill_bm(cfg). -7 unknown cfg, -2 K % r9k_moe_prefill_bk(cfg). */
int r9k_moe_4bit_prefill(int nv, long a, long as, long wq, long ws, long wref, long c, long sorted_ids,
                         long expert_ids, long ntpp, long topk_w, long ws_estride, long wref_estride, int max_blocks,
                         int numel, int a_row_div, int K, int N, int cfg, long stream);

/* Native NVFP4 experts: the same grouped GEMM over the checkpoint's e2m1 codes, e4m3 per-16 scales and a per-row fp32
 * multiplier wg (wg_estride floats per expert), exact; ws / wq in prepare_nvfp4_weights' layout (ws_estride bytes per
 * expert, code stride N * ceil(K/128) * 64 bytes). Decode-family tables (16 * MT-row blocks, MT 1 / 2 / 4). WV and
 * NPW are accepted and not used; K % (16 SK) as the reference's rule. 0, -1 N % 16, -2 K, -3 argument, -7 MT,
 * -6 launch error. Replaces kernels/r9k_moe_mxfp4a8.hip:641-647 (r9k_moe_nvfp4a8). */
int r9k_moe_nvfp4a8(long a, long as, long wq, long ws, long wg, long c, long sorted_ids, long expert_ids, long ntpp,
                    long topk_w, long ws_estride, long wg_estride, int max_blocks, int numel, int a_row_div, int K,
                    int N, int WV, int SK, int NPW, int MT, long stream);

/* Rows per routing block / K granularity of a prefill cfg (-1: no such cfg).
 * Replace kernels/r9k_moe_mxfp4a8.hip:1196-1203. */
int r9k_moe_prefill_bm(int cfg);
int r9k_moe_prefill_bk(int cfg);

/* Rows per M tile (16); the reference's Python asserts it. Replaces kernels/r9k_moe_mxfp4a8.hip:557. */
int r9k_moe_block(void);

/* 0: no folded-exponent kernels (the scaled MFMA applies the block exponents). Replaces :558. */
int r9k_fold_supported(void);

/* Per-row dynamic fp8 quant: x bf16 [M][K] (row stride ld) -> q e4m3fn [M][K], s fp32 [M] (amax / 448).
 * Replaces kernels/r9k_moe_mxfp4a8.hip:1745-1757. -3 bad shape, -6 launch error. */
int r9k_quant_rows_fp8(long x, long q, long s, int M, int K, int ld, long stream);

/* The same plus g[row] = bf16(sigmoid(bf16(x[row] . wg))) as fp32 (shared-expert gate); tiled != 0 (the gfx1201
 * fragment-tiled store) returns -3. Replaces kernels/r9k_moe_mxfp4a8.hip:1770-1781. */
int r9k_quant_rows_fp8_gate(long x, long q, long s, long wg, long g, int M, int K, int ld, int tiled, long stream);

/* silu(gate) * up + per-row fp8 quant: gu bf16 [M][2I] -> q e4m3fn [M][I], s fp32 [M].
 * Replaces kernels/r9k_moe_mxfp4a8.hip:550-555. */
int r9k_silu_mul_quant_fp8(long gu, long q, long s, int M, int I, long stream);

/* Softmax top-k routing + align tables in one call: logits bf16 [M][E] (row stride ldl) -> weights fp32 [M][topk],
 * ids int32 [M][topk], sorted_ids int32 [capacity], expert_ids int32 [capacity / blk], ntpp int32 [1]
 * (capacity = ceil((M*topk + E*(blk-1)) / blk) * blk). scratch: 2E+1 int32, zeroed once by the caller (reference contract);
 * scratch[0] is the workgroups' arrival counter and is left zero. Calls sharing one scratch must not overlap.
 * Tables in canonical order (rows ascending within each expert). Returns 0, 1 for an unsupported shape
 * (E > 1024, topk > 16, blk not a power of two), else the HIP error. Replaces kernels/r9k_moe_route.hip:217-233. */
int r9k_moe_route(long logits, int ldl, long weights, long ids, long sorted_ids, long expert_ids, long ntpp,
                  long scratch, int M, int E, int topk, int renorm, int blk, long stream);
int r9k_moe_route_max_experts(void);   /* 1024; replaces r9k_moe_route.hip:235 */
int r9k_moe_route_max_topk(void);      /* 16;   replaces r9k_moe_route.hip:236 */

/* Weighted top-k sum: out[m, n] = bf16(sum_j down[m, j, n] (+ shared[m, n])), fp32, j ascending, one rounding.
 * down bf16 [M][topk][N] contiguous, shared [M][N] (row stride ld_shared) or 0, out row stride ld_out; N % 8 == 0.
 * Replaces kernels/r9k_moe_sum.hip:62-69. */
int r9k_moe_sum(long down, long shared, long out, int M, int topk, int N, long ld_shared, long ld_out, long stream);

/* Router (gate) GEMM at decode widths: out[M][E] = x[M][K] bf16 . w[E][K]^T bf16 with fp32 accumulation, rounded
 * once to bf16 (out_bf16 = 1) or stored fp32; row strides sx / sw / so in elements. act_cols > 0 applies the
 * hyper-connection epilogue s = bf16(v) / hc, s / (1 + exp(-s)) to the first act_cols columns. Rules: 1 <= M <= 32,
 * E >= 1, K >= 8, split in {1, 2, 4, 8}, K % (8 split) == 0, sx and sw multiples of 8, x and w 16-byte aligned.
 * 0, or -1 M / E / K, -2 split, -3 K % (8 split), -4 strides or alignment, -7 act_cols with hc <= 0, -6 launch error.
 * Replaces kernels/r9k_router.hip:120-155 (r9k_router_gemm). */
int r9k_router_gemm(long x, long sx, long w, long sw, long out, long so, int M, int E, int K, int split, int out_bf16,
                    int act_cols, float hc, long stream);
int r9k_router_max_m(void);            /* 32; replaces r9k_router.hip:155 */

/* --- entry points with no reference C symbol ------------------------------------------------------------------ */

/* Routing only (the role of vLLM's topk_softmax behind the stock FusedTopKRouter, which the reference calls when
 * its fused router is off: r9700_vllm/moe/route.py:159-163). Same numerics as r9k_moe_route. 0 / 1 / HIP error. */
int r9k_moe_topk(long logits, int ldl, long weights, long ids, int M, int E, int topk, int renorm, long stream);

/* r9k_moe_topk plus r9k_quant_rows_fp8 of the layer's activations in ONE launch, any M (the work the reference does
 * in vLLM's topk_softmax and then r9k_quant_rows_fp8, r9700_vllm/moe/experts.py:185, at prefill widths): x bf16
 * [M][H] (row stride ldx) -> xq e4m3fn [M][H], xs fp32 [M], the bytes of r9k_quant_rows_fp8; weights / ids as
 * r9k_moe_topk. Top-k and quant workgroups alternate so each CU runs both. Returns 2 with nothing launched for H % 8,
 * H > 4096, ldx % 8 or misaligned x (16 bytes) / xq (8 bytes): then call the two entries. 1 bad arguments, else the
 * HIP error. */
int r9k_moe_topk_quant(long logits, int ldl, long weights, long ids, int M, int E, int topk, int renorm, long x,
                       long ldx, int H, long xq, long xs, long stream);

/* r9k_moe_route plus the per-token fp8 quant of the layer's activations in the same launch (the work the reference
 * does in r9k_moe_route and then r9k_quant_rows_fp8, r9700_vllm/moe/experts.py:185): x bf16 [M][H] (row stride
 * ldx) -> xq e4m3fn [M][H], xs fp32 [M], the bytes of r9k_quant_rows_fp8. scratch as for r9k_moe_route (its first
 * int is the arrival counter, used above 16 rows). Served while the routing is one launch (M * topk <= 4096) for
 * H % 8 == 0, H <= 4096, ldx % 8 == 0, x 16-byte and xq 8-byte aligned; any other shape returns 2 with nothing
 * launched (run r9k_moe_route + r9k_quant_rows_fp8 instead). 0 / 1 bad arguments / 2 / HIP error. */
int r9k_moe_route_quant(long logits, int ldl, long weights, long ids, long sorted_ids, long expert_ids, long ntpp,
                        long scratch, int M, int E, int topk, int renorm, int blk, long x, long ldx, int H, long xq,
                        long xs, long stream);

/* r9k_moe_route(_quant) with the tables in two layouts of which the device keeps one. No counterpart in the
 * reference, which picks the block size on the host from the row count (r9700_vllm/kernels/moe.py:532-535): a
 * skewed step the host cannot see may take the 256-row blocks. The per-expert counts decide: with nbig the number of
 * big_blk-row blocks, the big layout is kept when nbig > 0 and M * topk >= min_rows * nbig (r9k_moe_pick_blocks'
 * rule); only the kept layout is written (blk rows: sorted_ids / expert_ids over the whole capacity, ntpp; big_blk
 * rows: sorted_big / expert_big up to ntpp_big, the live entries), the other's ntpp is set to 0. x = 0: no
 * activation quant (else as r9k_moe_route_quant). Served for M * topk <= 4096 and, with x, rows the wave quant
 * takes; 2 otherwise (nothing launched). 0 / 1 bad arguments / 2 / HIP error. */
int r9k_moe_route_dual(long logits, int ldl, long weights, long ids, long sorted_ids, long expert_ids, long ntpp,
                       long scratch, int M, int E, int topk, int renorm, int blk, long x, long ldx, int H, long xq,
                       long xs, int big_blk, long sorted_big, long expert_big, long ntpp_big, int min_rows,
                       long stream);

/* Align tables only, from ids int32 [numel] (the role of vLLM's moe_align_block_size, called at
 * r9700_vllm/moe/experts.py:172 of the reference). ids outside [0, E) are left out. scratch: at least
 * r9k_moe_align_scratch_ints(numel, E) int32 (1 up to 4096 routed rows, else 16 + ceil(numel / 2048) * E): the
 * per-chunk histograms of the multi-workgroup path (rewritten by every call, so its contents at entry do not matter);
 * calls sharing one scratch must not overlap. */
int r9k_moe_align(long ids, int numel, int E, int blk, long sorted_ids, long expert_ids, long ntpp, long scratch,
                  long scratch_ints, long stream);
long r9k_moe_align_scratch_ints(int numel, int E);

/* No counterpart in the reference: r9k_moe_align writing only the live tables (the expert blocks up to ntpp, with
 * their padding entries); sorted_ids / expert_ids past ntpp are left as they were. For consumers that read no
 * further than ntpp, as this library's GEMMs: a 256-row layout at decode widths (numel + E * 255 entries, mostly
 * tail) costs a fraction to build. Arguments and return codes as r9k_moe_align. */
int r9k_moe_align_live(long ids, int numel, int E, int blk, long sorted_ids, long expert_ids, long ntpp,
                       long scratch, long scratch_ints, long stream);

/* No counterpart in the reference (it sends every expert through one block size picked on the host): the tables of
 * one routed step split by expert size on the device, for prefill steps whose routing leaves many experts with a
 * handful of rows. Experts with more than thr rows get blk_big-row blocks in (sorted_big, expert_big, ntpp_big), the
 * others blk_small-row blocks in the small tables; each table holds only its experts' rows (ascending within each
 * expert, as r9k_moe_align) and is written up to its ntpp only (as r9k_moe_align_live). Capacities and scratch as
 * r9k_moe_align's for each block size. 0 / 1 bad arguments or HIP error. */
int r9k_moe_align_split(long ids, int numel, int E, int thr, int blk_big, long sorted_big, long expert_big,
                        long ntpp_big, int blk_small, long sorted_small, long expert_small, long ntpp_small,
                        long scratch, long scratch_ints, long stream);

/* No counterpart in the reference. r9k_moe_align for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): no scratch argument, nothing allocated; the multi-workgroup
 * path uses the library's own file-scope device array (r9k_moe_align_noalloc_max_ints() int32 = 1 MiB per GPU, held
 * until the process ends; every call rewrites the histograms it reads). Every call on one GPU
 * shares that array: calls that overlap on one GPU race. Tables bit-identical to r9k_moe_align's. 0; 1 bad arguments
 * or HIP error; -9 the step needs more than r9k_moe_align_noalloc_max_ints() scratch ints (see
 * r9k_moe_align_scratch_ints); -6 the array's device address could not be obtained. */
int r9k_moe_align_noalloc(long ids, int numel, int E, int blk, long sorted_ids, long expert_ids, long ntpp,
                          long stream);
long r9k_moe_align_noalloc_max_ints(void);

/* The tail of a decode-width MoE layer in one launch: SiLU-gating + per-row fp8 quant of the gate_up output, the
 * grouped down GEMM with the router weight in its epilogue, and the weighted top-k sum (+ an optional shared-expert
 * term). Replaces, as one entry, kernels/r9k_moe_mxfp4a8.hip:550 (r9k_silu_mul_quant_fp8) + :631-638 (the down
 * r9k_moe_mxfp4a8 with a_row_div 1 and topk_w) + kernels/r9k_moe_sum.hip:62 (r9k_moe_sum). Token-major: no routing
 * tables, the expert of routed row t * topk + j is ids[t * topk + j] (outside [0, E): contributes 0).
 * gu bf16 [T * topk][2I]; ids int32 [T * topk]; tw fp32 [T * topk]; wq / ws the down weights (N = hidden, K = I) in
 * the r9k_moe_mxfp4a8 layout, ws_estride bytes per expert; shared bf16 [T][N] (row stride ld_shared) or 0; out bf16
 * [T][N] (row stride ld_out). Equals the three launches bit for bit for I < 1024. Served: I % 128 == 0, I <= 2048,
 * N % 16 == 0, topk <= 16 (I > 1024 with topk > 8 not); else 2 with nothing launched. 0, -3 bad argument, -6 launch
 * error. */
int r9k_moe_down_sum(long gu, long ids, long tw, long wq, long ws, long ws_estride, long shared, long ld_shared,
                     long out, long ld_out, int T, int topk, int E, int I, int N, long stream);

/* The grouped MXFP4 x fp8 GEMM over 16-row routing blocks as a block stream: one workgroup of 16 waves walks one
 * block's expert (or a wide column slice of it) over all of K, the block's activation rows staged once in LDS.
 * epi 0 replaces kernels/r9k_moe_mxfp4a8.hip:631-638 (r9k_moe_mxfp4a8 at MT = 1) with its values bit for bit at
 * its single-wave split: c bf16 [numel][N], topk_w optional, cs unused. epi 1 replaces, as one entry, the gate_up
 * r9k_moe_mxfp4a8 + :550 (r9k_silu_mul_quant_fp8): c e4m3 [numel][N / 2] = the per-row fp8 quant of
 * silu(gate) * up, cs fp32 [numel] its row scales, bit-equal to the two launches; topk_w must be 0. Tables in the
 * moe_align_block_size format with 16-row blocks; blocks_hint = the caller's bound on live blocks (min(E, numel)),
 * which sizes the column slices of epi 0. Served: K % 128 == 0, N % 16 == 0 (epi 1: N / 16 = 32 or 64), the staged
 * rows within 64 KB of LDS; else 2 with nothing launched. 0, -3 bad argument, -6 launch error. */
int r9k_moe_stream(int epi, long a, long as, long wq, long ws, long c, long cs, long sorted_ids, long expert_ids,
                   long ntpp, long topk_w, long ws_estride, int max_blocks, int numel, int a_row_div, int K, int N,
                   int blocks_hint, long stream);

/* gate_up, SiLU-gating + per-row fp8 quant and down of a decode-width MoE layer in one launch, one 16-row routing
 * block a workgroup (both GEMMs walk the same tables, so a block's down rows need only its own gate_up rows, handed
 * over in LDS). Replaces, as one entry, the gate_up kernels/r9k_moe_mxfp4a8.hip:631-638 (r9k_moe_mxfp4a8) + :550
 * (r9k_silu_mul_quant_fp8) + the down r9k_moe_mxfp4a8 with topk_w. a e4m3 [T][K1], as fp32 [T] (a_row_div = topk);
 * w1q / w1s the gate_up weights (N1 = 2I, K1), w2q / w2s the down weights (N2, K2 = I), in the r9k_moe_mxfp4a8 layout
 * (w?s_estride bytes per expert of the scale tensors); c bf16 [numel][N2] = the down rows, bit-equal to the three
 * launches at their single-wave split; the top-k sum follows (r9k_moe_sum). Served: K1 % 128 == 0, K1 <= 4096,
 * I % 128 == 0, I <= 1024, N2 % 32 == 0, the LDS within 96 KB, numel * N2 * 2 < 2^31; else 2 with nothing launched.
 * 0, -3 bad argument, -6 launch error. */
int r9k_moe_stream_layer(long a, long as, long w1q, long w1s, long w2q, long w2s, long c, long sorted_ids,
                         long expert_ids, long ntpp, long topk_w, long w1s_estride, long w2s_estride, int max_blocks,
                         int numel, int a_row_div, int K1, int N1, int N2, long stream);

/* The dense MXFP4 weight-only linear at decode widths in one launch: the per-row fp8 quant of the bf16 activations
 * (each workgroup quantises the M <= 4 rows into LDS) and the GEMM. Replaces, as one entry, the reference's
 * r9k_quant_rows_fp8 + r9k_moe_mxfp4a8 over identity tables (r9700_vllm/ops.py:89-117; kernels/r9k_moe_mxfp4a8.hip
 * :1745-1760, :631-638). x bf16 [M][K] (row stride ldx, 16-byte aligned); wq / ws one expert in the r9k_moe_mxfp4a8
 * layout; out bf16 [M][N] (row stride ldo). Bit-equal to the two launches. Served: 1 <= M <= 4, K % 128 == 0,
 * K <= 8192, N % 16 == 0; else 2 with nothing launched. 0, -3 bad argument, -6 launch error. */
int r9k_dense_mxfp4_qa(long x, long ldx, long wq, long ws, long out, long ldo, int M, int N, int K, long stream);

/* The GEMM of the same dense linear from activations already quantised (r9k_quant_rows_fp8's codes and row scales),
 * 1 <= M <= 16 rows, on the dense kernel's weight stream: the reference runs it as r9k_moe_mxfp4a8 over identity
 * tables (r9700_vllm/ops.py:89-117; kernels/r9k_moe_mxfp4a8.hip:631-638). q fp8 [M][K] (row stride ldq bytes, both
 * 16-byte aligned), s fp32 [M], tw fp32 [M] row weights or 0 (r9k_moe_mxfp4a8's topk_w: the shared expert's gate);
 * wq / ws one expert in the r9k_moe_mxfp4a8 layout; out bf16 [M][N] (row stride ldo). Bit-equal to r9k_moe_mxfp4a8.
 * Served: 1 <= M <= 16, K % 128 == 0, N % 16 == 0; else 2 with nothing launched. 0, -3 bad argument, -6 launch
 * error. */
int r9k_dense_mxfp4_a8(long q, long ldq, long s, long tw, long wq, long ws, long out, long ldo, int M, int N, int K,
                       long stream);

/* The native NVFP4 dense linear at decode widths in one launch: the per-row fp8 quant of the bf16 activations (each
 * workgroup quantises the M <= 2 rows into LDS) and the NVFP4 x fp8 GEMM. Replaces, as one entry, the reference's
 * r9k_quant_rows_fp8 + r9k_moe_nvfp4a8 over identity tables (r9700_vllm/ops.py:66-83; kernels/r9k_moe_mxfp4a8.hip
 * :641-647). x bf16 [M][K] (row stride ldx, 16-byte aligned); wq / ws / wg one expert in the layout of
 * r9k_moe_nvfp4a8; out bf16 [M][N] (row stride ldo). Bit-equal to the two launches. Served: 1 <= M <= 2,
 * K % 128 == 0, K <= 8192, N % 16 == 0; else 2 with nothing launched. 0, -3 bad argument, -6 launch error. */
int r9k_dense_nvfp4_qa(long x, long ldx, long wq, long ws, long wg, long out, long ldo, int M, int N, int K,
                       long stream);

/* Load-time NVFP4 -> MXFP4 with MSE-searched block exponents (the reference does this with torch:
 * r9700_vllm/quant/nvfp4.py:39-90). packed u8 [N][K/2], s16 e4m3 [N][K/16], row_div fp32 [N] -> out_packed u8
 * [N][K/2], out_e8m0 u8 [N][K/32] (checkpoint layout). -2 K % 32, -3 bad pointer / alignment, -6 launch error. */
int r9k_nvfp4_to_mxfp4(long packed, long s16, long row_div, long out_packed, long out_e8m0, int N, int K, long stream);

/* The same MSE search on fp32 weights [N][K] (r9700_vllm/quant/nvfp4.py:54-75, quantize_mxfp4_search). */
int r9k_quantize_mxfp4_search(long w, long out_packed, long out_e8m0, int N, int K, long stream);

/* Device-side block-size choice for one routed step whose tables were built in both layouts (16 * MT-row decode
 * blocks, big_blk-row prefill blocks): keeps the big layout when numel >= min_rows * (ntpp_big / big_blk) (the
 * touched experts' average rows, estimated from the big layout's block count), else the small one; the other gets
 * ntpp = 0, so the GEMMs launched over it exit at once. No reference counterpart (the reference picks on the host
 * from the row count, r9700_vllm/kernels/moe.py:532-535). 0, -1 bad arguments, -6 launch error. */
int r9k_moe_pick_blocks(long ntpp_small, long ntpp_big, int numel, int big_blk, int min_rows, long stream);

/* ---- Host-offloaded experts: device LRU cache (reference r9700_vllm/moe/cache.py:1-20, 182-395) ---- */

/* One manage step (replaces kernels/third_party/davetha/r4d_lru.hip:187-274, bound at moe/cache.py:39-41):
 * ids int32 [mk] (<0 or >= E ignored); table int32 [E] expert -> slot or -1; map_cold int32 [E] expert -> itself
 * when not resident else -1; slot_expert int32 [S]; slot_stamp int64 [S]; routed u8 [E] (out: this step's flags);
 * step int64 [1]; miss int32 [max_inserts][2] (out: (expert, slot) of each insert); n_miss int32 [1]. When more
 * than max_distinct experts are routed only step and routed change; otherwise resident routed experts are
 * restamped and the non-resident ones, in expert-id order and at most max_inserts, take the slots of the smallest
 * (stamp << 20 | slot) among slots whose expert is not routed. One workgroup, no atomics (deterministic).
 * -1 E <= 0 / E > 8192 / S <= 0 / S > 1024 / S > E / mk < 0, -2 max_inserts outside [0, S], -3 null pointer,
 * -4 int64 arrays not 8-byte aligned, -6 launch error. */
int r4d_lru_manage(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table, long map_cold,
                   long slot_expert, long slot_stamp, long routed, long step, long miss, long n_miss, long stream);

/* r4d_lru_manage, then in the same launch hot[i] = table[ids[i]], cold[i] = map_cold[ids[i]] (-1 for ids outside
 * [0, E)) from the updated maps: the routing ids of the resident and the host pass (the reference derives its two
 * align tables inside its fused manage kernel, r4d_lru.hip:305-631, bound at moe/cache.py:45-48). hot and cold
 * int32 [mk], both given or both 0. Codes as r4d_lru_manage. */
int r9k_lru_manage_map(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table, long map_cold,
                       long slot_expert, long slot_stamp, long routed, long step, long miss, long n_miss, long hot,
                       long cold, long stream);

/* The reference's one-launch manage + both moe_align_block_size outputs (replaces r4d_lru.hip:596-610, bound at
 * moe/cache.py:45-48 and called at :345-352): one manage step (as r4d_lru_manage), then the resident pass's tables
 * over slot ids (ids through the updated table) and the host pass's over expert ids (through map_cold), block size
 * bs, each in canonical order (rows ascending within an id). sorted_* int32 [L] (padding and tail = mk), eids_*
 * int32 [NB] (-1 past the end), npad_* int32 [1] = padded total. L must cover the padded total's bound (min(mk * bs,
 * mk + E (bs - 1)) while mk < E, else mk + E (bs - 1), vLLM's sizing) and NB * bs >= L. Served for E <= 1024 and
 * mk <= 4096 (one workgroup builds the tables); 2 otherwise (nothing launched). -1 sizes, other codes as
 * r4d_lru_manage. */
int r4d_lru_fused(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table, long map_cold,
                  long slot_expert, long slot_stamp, long routed, long step, long miss, long n_miss, int bs, int L,
                  int NB, long sorted_hot, long eids_hot, long npad_hot, long sorted_cold, long eids_cold,
                  long npad_cold, long stream);

/* r4d_lru_fused with this library's table capacity (sorted capacity(mk, E, blk) = ceil((mk + E (blk - 1)) / blk)
 * * blk entries, expert ids capacity / blk, as r9k_moe_align writes them); sorted_c = 0 skips the host pass's tables
 * (steps whose host pass is provably empty); hot_ids (int32 [mk], 0 = not wanted) receives each routed row's slot
 * (-1 = not resident), for the token-major decode tail over the slots. x != 0: the same launch writes the experts'
 * input quant, xq e4m3 [T][H] + xs fp32 [T] = r9k_quant_rows_fp8 of the T <= 64 bf16 rows of x (row stride ldx,
 * 16-byte aligned; H % 8 == 0, H <= 4096). No counterpart of its own in the reference (the same step as
 * r4d_lru_fused plus the quant the reference launches after it, moe/experts.py:167-199; bound by moe/cache.py
 * LayerCache.update_fused). 2 when not served (E > 1024 or mk > 4096: nothing launched, x not quantised); -7 quant
 * arguments out of range. */
int r9k_lru_manage_tables(long ids, int mk, int E, int S, int max_distinct, int max_inserts, long table, long map_cold,
                          long slot_expert, long slot_stamp, long routed, long step, long miss, long n_miss, int blk,
                          long sorted_h, long eids_h, long ntpp_h, long sorted_c, long eids_c, long ntpp_c,
                          long hot_ids, long x, long ldx, int H, int T, long xq, long xs, long stream);

/* Copy each listed expert's six per-expert slabs host -> slot (replaces r4d_lru.hip:276-303, bound at
 * moe/cache.py:42-44): slab i of expert e at s_i + e * b_i goes to d_i + slot * b_i for the first n_miss[0]
 * (expert, slot) pairs of miss. Bytes b_i multiples of 16 (0 = unused slab), pointers 16-byte aligned. Grid
 * (chunks, lanes) of 256-thread workgroups. -2 chunks / lanes outside [1, 65535], -3 null pointer, -4 size or
 * alignment, -6 launch error. */
int r4d_lru_gather(long d0, long s0, long b0, long d1, long s1, long b1, long d2, long s2, long b2, long d3, long s3,
                   long b3, long d4, long s4, long b4, long d5, long s5, long b5, long miss, long n_miss, int chunks,
                   int lanes, long stream);

/* hot[i] = table[ids[i]], cold[i] = map_cold[ids[i]] (-1 for ids outside [0, E)): the routing ids of the resident
 * and the host pass, for r9k_moe_align. The reference computes them inside its fused manage kernel
 * (r4d_lru.hip:305-631, moe/cache.py:336-354). -1 mk < 0 / E <= 0, -3 null pointer, -6 launch error. */
int r9k_lru_map_ids(long ids, int mk, int E, long table, long map_cold, long hot, long cold, long stream);

/* Cold staging (the reference's opt-in R9K_STAGE_COLD, moe/cache.py:358-393, built there with torch ops; no
 * counterpart as one entry): ids int32 [mk] (this step's routed experts), table int32 [E] (expert -> slot, -1 = host)
 * after this step's manage -> stage_map int32 [E] (each routed non-resident expert's staging index, in ascending
 * expert order; -1 otherwise), miss int32 [cap][2] ((expert, staging index) pairs for r4d_lru_gather), n_miss [1]
 * (their count, at most cap; with every slot filled at most E - S experts are cold). One workgroup, deterministic.
 * 0, -1 bad sizes (E > 8192), -3 null pointer, -6 launch error. */
int r9k_lru_stage_map(long ids, int mk, int E, long table, int cap, long stage_map, long miss, long n_miss,
                      long stream);

/* Mapped pinned host memory for the expert store (the role of the reference's UVA tensors, utils/hostmem.py):
 * hipHostMalloc(Mapped | Portable), returned only when its device address equals its host address; 0 on failure or
 * bytes <= 0. r9k_host_free: 0 / -6. */
long r9k_host_alloc(long bytes);
int r9k_host_free(long ptr);

#ifdef __cplusplus
}
#endif

#endif /* R9K_H */
