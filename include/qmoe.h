/* qmoe — MI355X (gfx950) W4A16 MoE expert path, C ABI of libqmoe.so.
 *
 * Conventions (mirroring the reference's ctypes kernels under kernels/ and
 * their Python wrappers under fnx/):
 *  - every pointer is a device pointer except where noted; the caller
 *    allocates all outputs and any workspace; the library never allocates,
 *    never synchronises, and launches asynchronously on `stream`
 *    (a hipStream_t), so calls can be captured in a HIP graph;
 *  - bf16 tensors are uint16 bit patterns; int4pack weights are int32 words
 *    [.., K, N/8] whose nibble j (bits 4j..4j+3, low first, two's
 *    complement) is column 8c+j (tools/repack_w4a16.py:38-70,
 *    ops/scripts/r37_w4a16_semantics.py:69-76);
 *  - return 0 on launch, QMOE_EINVAL (-1) for rejected shapes, QMOE_EWORKSPACE
 *    (-2) for a short workspace, QMOE_ESCRATCH (-3) for a shape beyond a fixed
 *    no-allocation scratch, or a positive hipError_t from the launch
 *    (kernels/reduce/reduce.cpp:64 returns -1 the same way);
 *  - `counters` is an int32 array that must be zero before the first call;
 *    the kernels that use it return it to zero, so one buffer per device
 *    serves all calls issued in stream order (calls overlapping on two
 *    streams of one device must use different buffers).
 */
#ifndef QMOE_H
#define QMOE_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- W4A16 GEMM: torch_npu.npu_weight_quant_batchmatmul(x, W, S,
 *      antiquant_group_size=gs) at fnx/engine.py:698-701 (and 358-364).
 *      y[M,N] = bf16(sum_k x[m,k] * q[k,n] * S[k/gs, n]), fp32 accumulation.
 *      x bf16 [M,K], w int4pack [K,N/8], scale bf16 [K/gs, N], y bf16 [M,N].
 */
/* M <= 4: split-K GEMV; the K-slices' partials travel as tagged words
 * through the mailbox of `counters` (at least qmoe_w4a16_gemm_counters(M, K,
 * N) int32 slots, shared with qmoe_moe_decode: the same epoch, so one array
 * serves both in stream order); qmoe_w4a16_gemm_workspace() is 0 (the
 * workspace arguments are ignored). */
size_t qmoe_w4a16_gemm_workspace(int M, int K, int N);
int qmoe_w4a16_gemm_counters(int M, int K, int N);
int qmoe_w4a16_gemv(const void* x, const void* w, const void* scale, void* y, int M, int K, int N,
                    int group_size, void* workspace, size_t workspace_bytes, void* counters, void* stream);
/* M > 4: MFMA GEMM on exact fp16 operands. K % 64 == 0, gs % 32 == 0, K/gs <= 56; the workspace
 * (qmoe_w4a16_gemm_mfma_workspace(M, K) bytes) holds the rows in fp16 and their exponents. */
size_t qmoe_w4a16_gemm_mfma_workspace(int M, int K);
int qmoe_w4a16_gemm_mfma(const void* x, const void* w, const void* scale, void* y, int M, int K, int N,
                         int group_size, void* workspace, size_t workspace_bytes, void* stream);

/* ---- Grouped GEMM: torch_npu.npu_grouped_matmul([x], [w],
 *      antiquant_scale=[s], group_list=ends, split_item=3, group_type=0)
 *      at fnx/engine.py:712-716, 744-753. Rows [ends[e-1], ends[e]) use
 *      expert e; empty experts allowed. x bf16 [R,K], w int4pack [E,K,N/8],
 *      scale bf16 [E,G,N], y bf16 [R,N]; K % 64 == 0, gs % 32 == 0, K/gs <= 56. The row-tile table (int32
 *      tile_expert/tile_row0/tile_rows [mtiles_max], tile_count [1]) is built
 *      on the GPU by qmoe_tiles_from_ends or qmoe_route_group. */
int qmoe_gemm_tile_rows(void);
int qmoe_max_row_tiles(int R, int E, int BM);
int qmoe_tiles_from_ends(const void* ends_i64, int E, int R, int BM, void* tile_expert, void* tile_row0,
                         void* tile_rows, void* tile_count, void* stream);
/* One single-row tile per id: row j of x uses expert ids[j] (int64 [k]), so
 * qmoe_grouped_gemm with mtiles_max = k computes the diagonal blocks of the
 * Cartesian down projection directly (ExpW4.apply_diag, fnx/engine.py:703-721,
 * whose FNX_DECODE_DN_GMM branch runs a grouped GEMM over k one-row groups).
 * Rows with an id outside [0, E) stay unwritten. */
int qmoe_tiles_from_ids(const void* ids, int k, int E, void* tile_expert, void* tile_row0, void* tile_rows,
                        void* tile_count, void* stream);
size_t qmoe_grouped_gemm_workspace(int R, int K);
int qmoe_grouped_gemm(const void* x, int R, int K, int N, int E, int gs, const void* w, const void* scale,
                      const void* tile_expert, const void* tile_row0, const void* tile_rows,
                      const void* tile_count, int mtiles_max, void* y, void* workspace, size_t workspace_bytes,
                      void* stream);

/* ---- Router: probs = softmax(fp32 logits); top-k by (logit desc, id asc);
 *      w = bf16(p / sum of selected p). fnx/engine.py:1810-1813.
 *      logits bf16 [T,E] (E <= 1024), idx int64 [T,k], w bf16 [T,k], k <= 16. */
int qmoe_router_topk(const void* logits, void* idx_out, void* w_out, int T, int E, int k, void* stream);

/* ---- Grouping glue: counts = bincount(ids), ends = cumsum (group_list),
 *      order = stable expert-major argsort of ids, inverse[order[p]] = p.
 *      fnx/engine.py:1816-1823 (argsort / scatter_add_ / cumsum) and
 *      1832-1843 (inverse). ids int64 [R]; outputs int64. Optionally also
 *      the grouped GEMM row-tile table for tile height BM (pass NULL
 *      tile_expert to skip). Workspace: qmoe_route_group_workspace(R, E). */
size_t qmoe_route_group_workspace(int R, int E);
int qmoe_route_group(const void* ids, int R, int E, void* counts, void* ends, void* order, void* inverse,
                     int BM, void* tile_expert, void* tile_row0, void* tile_rows, void* tile_count,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ---- Fused decode expert block for B = 1..4 tokens (FnLayer._moe b == 1
 *      branch, fnx/engine.py:1859-1891, r152 flags): router, gate_up of the
 *      de-duplicated selected experts read straight from the expert-major
 *      int4pack (replaces expert_gather.gather + WQBM, fnx/engine.py:691-699),
 *      SwiGLU (npu_swiglu, 1866), down projection of row j with expert j
 *      (replaces the Cartesian WQBM + diagonal, 1873 / 703-721) and the top-k
 *      combine fused into its epilogue (replaces moe_epilogue.merge 1874 /
 *      weighted_reduce.reduce 1884), with the shared merge (post_ops.moe_merge,
 *      1887) when shared/gate are non-NULL.
 *      x bf16 [B,H], logits bf16 [B,E], gu_w int4pack [E,H,2MI/8], gu_s bf16
 *      [E,H/gs_gu,2MI], dn_w [E,MI,H/8], dn_s [E,MI/gs_dn,H], shared bf16
 *      [B,H] or NULL, gate bf16 [B] or NULL; out bf16 [B,H], idx_out int64
 *      [B,k], w_out bf16 [B,k].
 *      qmoe_moe_decode is one launch: its down-projection workgroups load
 *      their weights while the gate_up workgroups run; partial sums, SwiGLU
 *      rows and weighted products travel between workgroups as tagged
 *      64-bit words through a mailbox in the counters array, and every wait
 *      for them is bounded. One token with H a multiple of 256 and MI of
 *      128 runs in workgroup groups pinned to one XCD each (gate_up
 *      partials stay in that XCD's L2; the down partials meet in combiner
 *      workgroups); the bits are the same as the two-launch form's. Of the qmoe_moe_decode_counters()
 *      slots, those below QMOE_DECODE_MAILBOX_BASE - 2 are counters returned
 *      to zero; slot QMOE_DECODE_MAILBOX_BASE - 2 is the array's launch
 *      epoch (owned by the library); slot QMOE_DECODE_MAILBOX_BASE - 1 is an
 *      error flag, set (and left set until qmoe_moe_decode_status clears it)
 *      if a wait ever timed out, in which case that call's outputs are
 *      wrong; from QMOE_DECODE_MAILBOX_BASE on come the mailbox words (zero
 *      before the first call, then owned by the library: words of earlier
 *      calls are never taken for the current one); -1 for shapes whose
 *      counters would not fit below the epoch. Epoch, flag and mailbox
 *      belong to the array: calls overlapping on two streams are independent
 *      when they pass different arrays. The workspace only receives
 *      inspection copies (qmoe_moe_decode_layout): pass NULL (and 0 bytes)
 *      for none. Shapes: B 1..4, k <= 16 <= E <= 1024, H a multiple of 32 up
 *      to 8192, MI a multiple of 32 up to 2048, gs_gu a multiple of 8
 *      dividing H, gs_dn a multiple of 16 dividing MI. */
#define QMOE_DECODE_MAILBOX_BASE 65536
size_t qmoe_moe_decode_workspace(int B, int k, int H, int MI);
int qmoe_moe_decode_counters(int B, int k, int H, int MI);
/* Host-side query of where the decode workspace keeps its routing plan
 * (int32: nunique, uexp[64], umult[64], utok[64][4], uslot[64][4], then fp32
 * w[4][16]), the SwiGLU rows act (bf16 [B*k unique slots][4][MI]) and the
 * weighted products prod (bf16 values held as fp32, [B][k][H]), for
 * inspection after a call. */
int qmoe_moe_decode_layout(int B, int k, int H, int MI, size_t* off_plan, size_t* off_act, size_t* off_prod);
int qmoe_moe_decode(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                    const void* dn_s, const void* shared, const void* gate, void* out, void* idx_out,
                    void* w_out, int B, int E, int k, int H, int MI, int gs_gu, int gs_dn, void* workspace,
                    size_t workspace_bytes, void* counters, void* stream);
/* The same decode block (fnx/engine.py:1803-1891, as qmoe_moe_decode) with
 * decode-tile copies of the two projections' weights (gu_t, dn_t, both or
 * neither; from qmoe_decode_tiles_gate_up / _down, built with the same gs_gu;
 * 16-byte aligned).
 * The one-token launch on XCD groups then reads every workgroup's 16 KB of
 * weights in one contiguous block; other shapes use gu_w / dn_w. Same bits as
 * qmoe_moe_decode. */
int qmoe_moe_decode_tiled(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                          const void* dn_s, const void* gu_t, const void* dn_t, const void* shared, const void* gate,
                          void* out, void* idx_out, void* w_out, int B, int E, int k, int H, int MI, int gs_gu,
                          int gs_dn, void* workspace, size_t workspace_bytes, void* counters, void* stream);
/* The whole one-token MoE block after its fused shared/router projection
 * (fnx/engine.py:1786-1891 for b == 1): the routed experts as
 * qmoe_moe_decode_tiled, and in the same launch the shared expert's down
 * projection sh = bf16(bf16(bf16(silu(g)) * u) . sh_dn^T) from the projection
 * row sh_gu (bf16 [2 MI + 1]: gate | up | gate2, 16-byte aligned; sh_dn bf16
 * [H, MI]), merged as qmoe_moe_decode merges `shared` with gate = sh_gu[2 MI].
 * The same bits as qmoe_bf16_gemv_swiglu followed by qmoe_moe_decode. Takes
 * only the one-token launch on XCD groups (H a multiple of 256, MI of 128 and
 * at most 2048, E a multiple of 8, x and logits 16-byte aligned); QMOE_EINVAL
 * otherwise, and the caller runs the two launches. gu_t/dn_t may be NULL. */
int qmoe_moe_block_decode(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                          const void* dn_s, const void* gu_t, const void* dn_t, const void* sh_gu, const void* sh_dn,
                          void* out, void* idx_out, void* w_out, int E, int k, int H, int MI, int gs_gu, int gs_dn,
                          void* counters, void* stream);
/* Decode tiles of a layer's experts, a load-time copy beside the int4pack
 * container (fnx/engine.py:641-651, expert-major [E, K, N/8]) in the order
 * the one-token launch's workgroups read it: gate_up gu_w [E, H, 2 MI / 8] ->
 * gu_t of the same size; down dn_w [E, MI, H / 8] -> dn_t of the same size.
 * H a multiple of 256, MI of 128; gs_gu is the gate_up group size the decode
 * will be called with. */
int qmoe_decode_tiles_gate_up(const void* gu_w, void* gu_t, int E, int H, int MI, int gs_gu, void* stream);
int qmoe_decode_tiles_down(const void* dn_w, void* dn_t, int E, int H, int MI, void* stream);
/* Reads the error flag of a decode counters array into *flag_out (host
 * int: 1 if a bounded wait of some earlier call timed out, else 0) and, when
 * clear != 0, resets it; counters == NULL names the current device's
 * no-allocation scratch (qmoe_moe_decode_noalloc). Unlike every other entry
 * point this one synchronises `stream` (call it outside graph capture). The
 * reference has no counterpart: its operators report failures through their
 * return codes (fnx/weighted_reduce.py:40-41). */
int qmoe_moe_decode_status(const void* counters, int clear, int* flag_out, void* stream);
/* Workgroup placement of the current device. The one-token XCD-group decode
 * launch (and qmoe_moe_block_decode) and the one-row GEMV hand partial sums
 * between workgroups through one XCD's L2, which needs workgroup b of a
 * launch to run on XCD (b + c) mod 8. The first call that needs it (outside
 * graph capture) runs a probe kernel on `stream`, reads every workgroup's
 * XCC_ID back (synchronising) and keeps the verdict per device; a device that
 * fails, or is not yet probed while its stream is captured, runs the
 * device-coherent forms (same outputs, slower). mode 0: probe if needed and
 * return 1 (placement holds) or 0; mode 1: treat this device as failing from
 * now on; mode 2: forget the verdict (probe again on next use); modes 1 and
 * 2 return 0. No counterpart in the reference (its NPU kernels do not
 * depend on core placement). */
int qmoe_xcd_placement(int mode, void* stream);
/* qmoe_moe_decode with no workspace and no counters argument: it allocates
 * nothing (no hipMalloc, no allocating library call), for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid it). No counterpart in the reference. Its counters,
 * epoch, error flag and mailbox live in a fixed device array of
 * qmoe_moe_decode_noalloc_max_bytes() bytes (8 MiB) per GPU, held until the
 * process ends; shapes whose qmoe_moe_decode_counters() exceed it return
 * QMOE_ESCRATCH (-3) without launching (k = 10 fits up to H 4096 / MI 1024
 * for one token and up to H 3072 / MI 768 for four). Every call on a GPU shares that GPU's array: calls issued in
 * stream order are safe, calls that overlap on two streams of one GPU race.
 * The stream must belong to the current device. Same outputs as
 * qmoe_moe_decode, bit for bit. */
size_t qmoe_moe_decode_noalloc_max_bytes(void);
int qmoe_moe_decode_noalloc(const void* x, const void* logits, const void* gu_w, const void* gu_s, const void* dn_w,
                            const void* dn_s, const void* shared, const void* gate, void* out, void* idx_out,
                            void* w_out, int B, int E, int k, int H, int MI, int gs_gu, int gs_dn, void* stream);
/* The two launches qmoe_moe_decode makes, for callers that time or
 * interleave them: router + gate_up + SwiGLU (replaces expert_gather.gather +
 * WQBM + npu_swiglu, fnx/engine.py:1861-1866), then down + combine (replaces
 * the Cartesian WQBM + moe_epilogue.merge, 1873-1874). Same workspace and
 * counters; the second must follow the first on the same stream. */
int qmoe_moe_decode_gate_up(const void* x, const void* logits, const void* gu_w, const void* gu_s, void* idx_out,
                            void* w_out, int B, int E, int k, int H, int MI, int gs_gu, void* workspace,
                            size_t workspace_bytes, void* counters, void* stream);
int qmoe_moe_decode_down(const void* dn_w, const void* dn_s, const void* shared, const void* gate, void* out, int B,
                         int k, int H, int MI, int gs_dn, void* workspace, size_t workspace_bytes, void* counters,
                         void* stream);

/* ---- Grouped prefill expert block after routing (FnLayer._moe b > 1 branch
 *      with FNX_MOE_GROUP=1, fnx/engine.py:1825-1853): gate_up grouped GEMM
 *      on rows x[order[p] / k] (replaces x2.index_select + apply_grouped,
 *      1825-1826) with SwiGLU fused, down grouped GEMM with the routing
 *      weight folded into its epilogue and scattered to token-major rows, then
 *      the ordered slot sum (replaces the inverse + weighted_reduce mode 2,
 *      1832-1846), + shared (bf16 add, 1853) when non-NULL.
 *      wts bf16 [T*k], order int64 [T*k], tile table from qmoe_route_group.
 *      Workspace: qmoe_moe_prefill_workspace(T, k, H, MI). */
size_t qmoe_moe_prefill_workspace(int T, int k, int H, int MI);
/* Byte offsets in that workspace of the SwiGLU rows act (bf16 [T*k][MI],
 * expert-major row order) and the weighted down products prod (bf16
 * [T*k][H], token-major), for inspection after a call. */
int qmoe_moe_prefill_layout(int T, int k, int H, int MI, size_t* off_act, size_t* off_prod);
int qmoe_moe_experts_grouped(const void* x, int T, int H, int MI, int E, int k, const void* wts,
                             const void* order, const void* gu_w, const void* gu_s, int gs_gu,
                             const void* dn_w, const void* dn_s, int gs_dn, const void* tile_expert,
                             const void* tile_row0, const void* tile_rows, const void* tile_count,
                             int mtiles_max, const void* shared, void* out, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ---- fnx_gather_pair (kernels/expert_gather/gather.cpp:24-27, wrapper
 *      fnx/expert_gather.py:9-31): ow[kk, j*N/8 + c] = w4[ids[j], kk, c],
 *      os[g, j*N + n] = S[ids[j], g, n]. Any K, G, E, k; N % 32 == 0. */
int qmoe_expert_gather(const void* w4, const void* scales, const void* ids, void* ow, void* os, int K, int G,
                       int N, int E, int k, void* stream);
/* The same gather from the K-major artifact w4 int32 [K,E,N/8] (scales still
 * expert-major [E,G,N], the scale cache): ow[kk, j*N/8 + c] = w4[kk, ids[j], c].
 * Replaces ExpW4._wcat / _scat's index_select + reshape (fnx/engine.py:672-689). */
int qmoe_expert_gather_kmajor(const void* w4, const void* scales, const void* ids, void* ow, void* os, int K, int G,
                              int N, int E, int k, void* stream);

/* ---- fnx_weighted_reduce modes 1/2 (kernels/reduce/reduce.cpp:59-70, wrapper
 *      fnx/weighted_reduce.py:10-42): out[t,:] = bf16(sum_g bf16(x[row,:] *
 *      w[t,g])) in g order, row = inverse[t*G+g] (inverse non-NULL) or t*G+g.
 *      w is fp32 [B,G]; any width. Rows outside [0, nrows) contribute zero. */
int qmoe_weighted_reduce(const void* x, const void* w_f32, const void* inverse, void* out, int B, int G, int W,
                         long row_stride, long nrows, void* stream);

/* ---- fnx_moe_epilogue (kernels/moe_epilogue/epilogue.cpp:41-43, wrapper
 *      fnx/moe_epilogue.py:6-21): diagonal of cart [k, k*H], ordered bf16
 *      product sum, optional shared merge (shared/gate NULL: none). */
int qmoe_moe_epilogue(const void* cart, const void* w, const void* shared, const void* gate, void* out, int k,
                      int H, void* stream);

/* ---- fnx_moe_merge (kernels/post_ops/post_ops.cpp:91-94, wrapper
 *      fnx/post_ops.py:36-39): out = bf16(e + bf16(s * bf16(sigmoid(g)))). */
int qmoe_moe_merge(const void* e, const void* s, const void* gate, void* out, int B, int W, void* stream);

/* ---- npu_swiglu(gu.float(), dim=-1).to(bf16) (fnx/engine.py:1827, 1866):
 *      act[r, i] = bf16(silu(gu[r, i]) * gu[r, MI + i]). */
int qmoe_swiglu(const void* gu, void* act, int rows, int MI, void* stream);

/* ---- Artifact conversion (load time). The LQP expert layout to the W4A16
 *      container: tools/repack_w4a16.py:58-76 (unpack v2o, transpose, int4pack
 *      via npu_convert_weight_to_int4pack) and tools/repack_w4_em.py:16-19
 *      (the expert-major permute), with the scale cache of
 *      fnx/engine.py:653-659.
 *      v2o uint8 [E,N,K/2] (byte 64s+j of a row: low nibble W[128s+j]+8, high
 *      nibble W[128s+64+j]+8) -> w4 int32 int4pack [E,K,N/8] (expert_major
 *      != 0) or [K,E,N/8]. K % 128 == 0, N % 8 == 0, both pointers 16-byte
 *      aligned. */
int qmoe_lqp_to_int4pack(const void* v2o, void* w4, int E, int N, int K, int expert_major, void* stream);
/* s8 int8 [E,N,G], base fp16 [E,N] -> s8t int8 [G,E,N], base bf16 [E,N]
 * (round to nearest even), scales bf16 [E,G,N] = bf16(s8 * base_bf16); any
 * of the three outputs may be NULL (not written). */
int qmoe_lqp_scales(const void* s8, const void* base_fp16, void* s8t, void* base_bf16, void* scales, int E, int N,
                    int G, void* stream);
/* Scale cache of the W4A16 container from its artifact form (ExpW4.__init__ with
 * FNX_W4_SCALE_CACHE=1, fnx/engine.py:653-659): s8t int8 [G,E,N], base bf16
 * [E,N] -> scales bf16 [E,G,N] = bf16(bf16(s8t[g,e,n]) * base[e,n]). */
int qmoe_scale_cache(const void* s8t, const void* base_bf16, void* scales, int G, int E, int N, void* stream);

/* ---- Shared expert and router projection (fnx/engine.py:1786-1802, the
 *      fused sh_gu form of fnx/engine.py:1226-1241): F.linear on bf16 (the
 *      reference's _fl, fnx/engine.py:256), y[m,n] = bf16(sum_k a[m,k] *
 *      w[n,k]) with fp32 accumulation; w bf16 [N,K] row-major. 1 <= M <= 4,
 *      K % 8 == 0, K <= 4096; a row m of x starts at x + m*ldx, of y at
 *      y + m*ldy (ldx % 8 == 0). */
int qmoe_bf16_gemv(const void* x, long ldx, const void* w, void* y, long ldy, int M, int K, int N, void* stream);
/* The same projection with the output columns n >= split written to a second
 * matrix, y2[m*ldy2 + n - split]: the router logits of the fused projection
 * (logits = gu[:, 2MI+1:], fnx/engine.py:1786, 1795) as their own rows, so
 * the decode kernels read them 16-byte aligned. 0 <= split <= N, ldy >= split,
 * ldy2 >= N - split (y2 unused when split == N). */
int qmoe_bf16_gemv_split(const void* x, long ldx, const void* w, void* y, long ldy, void* y2, long ldy2, int split,
                         int M, int K, int N, void* stream);
/* The same projection for any number of rows on bf16 MFMA (the prefill form
 * of fnx/engine.py:1786-1802, which the reference runs as a plain torch
 * GEMM): K % 32 == 0, ldx % 8 == 0, x and w 16-byte aligned, any M and N
 * with x's and w's extents ((M-1)*ldx + K and N*K elements) under 2^30. */
int qmoe_bf16_gemm(const void* x, long ldx, const void* w, void* y, long ldy, int M, int K, int N, void* stream);
/* The same with the shared expert's SwiGLU as the activations, read from the
 * first projection gu: a[m,k] = bf16(bf16(silu(gu[m,k])) * gu[m,MI+k])
 * (F.silu(gu[:, :MI]) * gu[:, MI:2MI], fnx/engine.py:1788); K = MI. */
int qmoe_bf16_gemv_swiglu(const void* gu, long ldgu, const void* w, void* y, long ldy, int M, int MI, int N,
                          void* stream);
/* act[r, i] = bf16(bf16(silu(gu[r, i])) * gu[r, MI + i]), rows of gu ldgu apart. */
int qmoe_swiglu_bf16(const void* gu, long ldgu, void* act, long rows, int MI, void* stream);
/* out[r, c] = bf16(bf16(sigmoid(gate[r*ldg])) * sh[r, c]): torch.sigmoid(gate2) * sh
 * (fnx/engine.py:1793); sh and out bf16 [rows, H]. */
int qmoe_shared_gate(const void* sh, const void* gate, long ldg, void* out, long rows, int H, void* stream);

/* ---- W8A16 GEMM: npu_weight_quant_batchmatmul with int8 weights, the dense
 *      projections' op (DenseW8, fnx/engine.py:297-384, call at 358-364).
 *      y[M,N] = bf16(sum_k x[m,k] * q[k,n] * S[k/gs, n]), fp32 accumulation.
 *      x bf16 [M,K], w int8 [K,N], scale bf16 [K/gs, N], y bf16 [M,N];
 *      N % 16 == 0. */
/* M <= 4: split-K GEMV; K % 4 == 0, gs % 4 == 0; needs
 * qmoe_w8a16_gemv_workspace() bytes (when K > 64) and
 * qmoe_w8a16_gemv_counters(N) counter slots. */
size_t qmoe_w8a16_gemv_workspace(int M, int K, int N);
int qmoe_w8a16_gemv_counters(int N);
int qmoe_w8a16_gemv(const void* x, const void* w, const void* scale, void* y, int M, int K, int N, int group_size,
                    void* workspace, size_t workspace_bytes, void* counters, void* stream);
/* Any M: bf16 MFMA on 64 x 64 tiles, the group scales applied to per-group
 * sums; K % 32 == 0, gs % 32 == 0. */
int qmoe_w8a16_gemm_mfma(const void* x, const void* w, const void* scale, void* y, int M, int K, int N,
                         int group_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QMOE_H */
