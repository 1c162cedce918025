/*
 * moe_mi355.h -- C ABI of the MI355X (gfx950) MoE hot-path library
 * (libmoe_mi355.so).
 *
 * Conventions
 *  - Every pointer argument is a device pointer unless stated otherwise; the
 *    caller owns all memory, including the workspace (size it with the
 *    matching *_workspace() query).  The library never allocates device
 *    memory and keeps no reference to any buffer after the call returns.
 *  - `stream` is a hipStream_t passed as void*; all work is enqueued on it
 *    and nothing synchronises the host.
 *  - Return value: 0 on success, a negative MOE_E* code for a bad argument,
 *    or a positive hipError_t from a failed launch.  moe_last_error() returns
 *    the message of the last failure on the calling thread.
 *  - Element types: MOE_F32 (float32) and MOE_BF16 (bfloat16, raw bits).
 *    Index tensors are int64 (torch.long) unless named *_i32.
 *
 * Reference paths below are relative to moe-engine/ in the reference tree.
 */
#ifndef MOE_MI355_H
#define MOE_MI355_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum moe_dtype { MOE_F32 = 0, MOE_BF16 = 1 };

enum moe_status {
  MOE_OK = 0,
  MOE_EINVAL = -1,   /* bad shape / dtype / pointer argument */
  MOE_EWORKSPACE = -2 /* workspace smaller than the *_workspace() query */
};

/* Number of float slots in the router `stats` output before the per-expert
 * mean-probability block.  Layout of stats[MOE_STATS_HEAD + E]:
 *   [0] z_stat      mean_t (logsumexp_e logits[t,e])^2
 *   [1] aux_raw     E * sum_e (cnt_e / (N K)) * (mean_t p[t,e])
 *   [2] imbalance   max(cnt) / mean(cnt), 1.0 if mean(cnt) < 1e-9
 *   [3] cnt_mean    mean(cnt)
 *   [4] cnt_std     unbiased standard deviation of cnt
 *   [5] cnt_total   sum(cnt)  (== N*K when every slot was dispatched)
 *   [6] nonfinite   number of non-finite logits
 *   [7] dead        number of experts with cnt == 0
 *   [8 + e]         mean_t p[t,e]
 */
#define MOE_STATS_HEAD 8

const char* moe_version(void);
int moe_last_error(char* buf, size_t len);

/* Optional per-kernel timing for benchmarks (no counterpart in the
 * reference, which times its Triton launch with CUDA events inside the hot
 * path, pkg/kernels/moe_router.py L:313-343).  Off by default; when on, every
 * kernel launch is bracketed by two hipEvents recorded on its stream.
 * moe_prof_enable(1) clears the records and starts recording,
 * moe_prof_enable(0) stops recording and keeps them.  moe_prof_summary() waits for
 * the recorded events of `kernel` (NULL = all kernels) and returns the launch
 * count and total milliseconds.  moe_prof_kernel_name(i, ...) copies the i-th
 * distinct kernel name seen (launch order) and returns 1, or 0 past the end. */
int moe_prof_enable(int on);
int moe_prof_summary(const char* kernel, int64_t* launches, double* total_ms);
int moe_prof_kernel_name(int64_t i, char* buf, size_t len);

/* MFMA ceiling of the current device (bench only; no counterpart in the
 * reference): one block of 8 waves per CU runs `iters` x 4 independent chains
 * of the grouped GEMM's MFMA with no memory traffic, timed with hipEvents on
 * the null stream.  mode bit 0: the instruction (0: bf16 32x32x16; 1: e4m3
 * 32x32x64); bit 1: the operands (0: one near-constant fragment pair; 1: four
 * hashed fragment pairs re-paired on every MFMA, so the register data changes
 * as in a data-carrying GEMM -- the part's power limit then sets a lower
 * clock).  `iters` is rounded up to a multiple of 4.  Returns the dense rate
 * in TFLOP/s and the shader clock under that load in MHz (s_memtime ticks per
 * 100 MHz s_memrealtime tick).  Allocates and synchronizes. */
int moe_prof_mfma_ceiling(int64_t iters, int mode, double* tflops, double* clock_mhz);

/* HBM ceiling of the current device (bench only; no counterpart in the
 * reference): 10 timed grid-stride streams of 16-byte non-temporal accesses
 * (8 blocks of 256 threads per CU) over fresh buffers: mode 0 reads `bytes`,
 * 1 writes `bytes`, 2 copies `bytes` (2x moved), 3 reads bytes/4096 rows of
 * 4 KB once and writes each to 6 rows (7x moved: the permute's shape at K = 6).
 * Returns the moved bytes per second in GB/s.  Allocates and synchronizes. */
int moe_prof_hbm_ceiling(int64_t bytes, int mode, double* gbps);

/* ------------------------------------------------------------------------
 * Router forward: logits = x @ wg (+ bias), p = softmax(logits), top-k of p
 * (descending, exact ties -> lower expert index), w = v / max(sum v, 1e-30),
 * dispatch counts and the router statistics above.
 *
 * Replaces _triton_forward / _router_fwd_kernel
 * (pkg/kernels/moe_router.py L:297-388, L:102-176) and the per-forward
 * bookkeeping of MoERouter.forward: bincount (L:690), z-loss (L:603-612,
 * L:727-733), load imbalance (L:594-600), count mean/std (L:736-745).
 *
 *   x        [N, H]  x_dtype          wg [H, E] wg_dtype      bias [E] f32 or NULL
 *   idx_out  [N, K]  int64            w_out [N, K] w_dtype
 *   logits_out [N, E] f32             lse_out [N] f32
 *   cnt_out  [E] int64                stats_out [MOE_STATS_HEAD + E] f32
 *   aux_out  [1] f32 or NULL: aux_coef * stats[1] (load-balance loss)
 *   z_out    [1] f32 or NULL: z_coef * stats[0]   (z-loss)
 * Limits: 1 <= K <= min(E, 32), 1 <= E <= 256.
 * Workspace: zero it before its first use and reuse it for later calls on
 * the same stream.  Its first word is a completion counter that the call
 * expects at zero and leaves at zero (no other part of the library writes
 * it); calls that share a workspace must not overlap.
 * ---------------------------------------------------------------------- */
size_t moe_router_fwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype, int wg_dtype);
/* LDS bytes per workgroup of the forward kernel a call with these sizes and dtypes launches (-1 if the runtime
 * cannot report it): the figure MoERouter reports as RouterProfile.sram_bytes_per_block, in place of the Triton
 * tile estimate sram_bytes = 64 * BLOCK_E * dsize * 3 (pkg/kernels/moe_router.py L:380). */
int64_t moe_router_fwd_lds_bytes(int64_t N, int64_t H, int64_t E, int x_dtype, int wg_dtype);
int moe_router_fwd(const void* x, int x_dtype, const void* wg, int wg_dtype, const float* bias,
                   int64_t N, int64_t H, int64_t E, int64_t K,
                   int64_t* idx_out, void* w_out, int w_dtype,
                   float* logits_out, float* lse_out, int64_t* cnt_out, float* stats_out,
                   float aux_coef, float z_coef, float* aux_out, float* z_out,
                   void* workspace, size_t ws_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Router backward.  G = dL/dlogits [N, E] from
 *   (a) the top-k/renormalise term for upstream grad_w (NULL = zero),
 *   (b) aux_coef * grad_aux * d(aux_raw)/dlogits   (grad_aux NULL = 1.0),
 *   (c) z_coef   * grad_z   * d(z_stat)/dlogits    (grad_z   NULL = 1.0),
 * then dx = G @ wg^T (x_dtype) and dwg = x^T @ G (wg_dtype).  With bf16
 * tokens G is rounded to bf16 before the two products, as the reference does
 * (grad_logits.to(tokens.dtype)).
 *
 * Replaces _router_bwd_kernel and MoERouterFunction.backward
 * (pkg/kernels/moe_router.py L:178-251, L:504-553; fp64 form L:274-291).
 * The aux / z terms have no counterpart in the reference (its z-loss is a
 * detached float, L:603-612): d(aux_raw)/dl[t,j] = (E/N) p[t,j] (f_j - sum_e
 * p[t,e] f_e) with f = cnt/(N K), d(z_stat)/dl[t,j] = (2/N) lse_t p[t,j].
 * ---------------------------------------------------------------------- */
size_t moe_router_bwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype, int wg_dtype);
int moe_router_bwd(const void* x, int x_dtype, const void* wg, int wg_dtype,
                   const float* logits, const int64_t* idx, const void* grad_w, int gw_dtype,
                   const int64_t* cnt, const float* grad_aux, const float* grad_z,
                   float aux_coef, float z_coef,
                   int64_t N, int64_t H, int64_t E, int64_t K,
                   void* dx_out, void* dwg_out,
                   void* workspace, size_t ws_bytes, void* stream);
/* The router backward with the rest of x's gradient folded in: dx_out = G @ wg^T + dx_add, where dx_add
 * [N, H] (x_dtype, must not overlap dx_out) is the gradient of x from the layer's other consumer of the
 * tokens, the expert path.  In the reference autograd sums the two contributions to x.grad, the router's
 * (moe_router.py L:545-546) and the dispatch's (moe_layer.py L:317-319 via index/repeat_interleave), in a
 * separate addition; here the sum is formed in the dx stores (bf16: both rounded values added in fp32 and
 * rounded once, as that addition does).  Otherwise identical to moe_router_bwd. */
int moe_router_bwd_acc(const void* x, int x_dtype, const void* wg, int wg_dtype,
                       const float* logits, const int64_t* idx, const void* grad_w, int gw_dtype,
                       const int64_t* cnt, const float* grad_aux, const float* grad_z,
                       float aux_coef, float z_coef,
                       int64_t N, int64_t H, int64_t E, int64_t K,
                       const void* dx_add, void* dx_out, void* dwg_out,
                       void* workspace, size_t ws_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Dispatch planner.  From the router's idx [N, K] (int64) builds, on the
 * device and deterministically:
 *   drop_out [N, K] uint8  per-top-k-column capacity drops: slot (t, k) is
 *            dropped when t is at position >= capacity among the tokens whose
 *            k-th choice is the same expert (capacity < 0: no dropping,
 *            drop_out may be NULL);
 *   row_slot [N*K] int32   slot t*K+k held by each permuted row (-1: none);
 *   slot_row [N*K] int32   row of each slot (-1: the slot has no row);
 *   offsets  [E+1] int32   rows of expert e are [offsets[e], offsets[e+1]);
 *            rows >= offsets[E] are never computed;
 *   ndrop    [1] int32     number of dropped slots.
 * layout 0 ("reference") reproduces DistributedMoELayer.forward at ep=1: rows
 * are the tokens stable-sorted by their first choice, each repeated K times,
 * cut into E equal chunks of max(1, N*K / E) rows; dropped slots keep their
 * row and get zero weight.  layout 1 ("routed"): slot (t, k) goes to expert
 * idx[t, k], rows grouped by expert in slot order, dropped slots get no row.
 *
 * Replaces _cumcount and compute_capacity_drop_mask
 * (pkg/distributed/moe_layer.py L:64-115, L:118-155), the capacity rule of
 * L:300-306, the sort/repeat of L:317-319 and the chunking of L:327-336.
 * ---------------------------------------------------------------------- */
size_t moe_plan_workspace(int64_t N, int64_t K, int64_t E);
int moe_plan(const int64_t* idx, int64_t N, int64_t K, int64_t E, int64_t capacity, int layout,
             uint8_t* drop_out, int32_t* row_slot, int32_t* slot_row, int32_t* offsets, int32_t* ndrop,
             void* workspace, size_t ws_bytes, void* stream);

/* Allocation-free planner (no counterpart in the reference: for callers that cannot allocate device memory
 * or take a workspace -- code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, outputs and errors as moe_plan without the workspace: the planner's block
 * tables go to a fixed device array of MOE_PLAN_SCRATCH_BYTES inside the library, which each GPU the
 * library runs on holds until the process ends.  Shapes whose tables exceed it (moe_plan_workspace(N, K, E)
 * > MOE_PLAN_SCRATCH_BYTES; e.g. N*K > 2^21 slots at K*E = 1024 keys) are rejected with MOE_EINVAL.  The
 * array needs no initialisation (every table is written before it is read) and keeps the last call's
 * contents.  Every call on one GPU shares that GPU's array: calls that overlap on one GPU (different
 * streams, different host threads) race; serialise them.  Call it with the stream's device current. */
#define MOE_PLAN_SCRATCH_BYTES (8 << 20)
int moe_plan_noalloc(const int64_t* idx, int64_t N, int64_t K, int64_t E, int64_t capacity, int layout,
                     uint8_t* drop_out, int32_t* row_slot, int32_t* slot_row, int32_t* offsets, int32_t* ndrop,
                     void* stream);

/* _cumcount for any int64 group ids (pkg/distributed/moe_layer.py L:64-115): out[i] = the number of j < i
 * with groups[j] == groups[i].  moe_plan computes the same for ids that fit its key tables (one contiguous
 * range of at most 1024 values); this entry point takes every other input (any range, any number of distinct
 * ids, negative ids): a stable radix sort of (id, position) pairs (rocPRIM), each element's rank being its
 * sorted position minus the first sorted position of its id.  n <= 2^31 - 1.  Not for graph capture (the sort
 * clears its counters with hipMemsetAsync). */
size_t moe_cumcount_workspace(int64_t n);
int moe_cumcount(const int64_t* groups, int64_t n, int64_t* out, void* workspace, size_t ws_bytes, void* stream);

/* Permute (dispatch): xp[slot_row[t*K+k]] = x[t] for every slot whose row is computed (0 <= row <
 * offsets[E]); other rows of xp are left unwritten.  Rows are row_bytes long (a multiple of 16); each token
 * row is read once and written to its K rows.  Replaces flat[sort_order].repeat_interleave(K)
 * (pkg/distributed/moe_layer.py L:318-319). */
int moe_permute(const void* x, int64_t row_bytes, const int32_t* slot_row, const int32_t* offsets,
                int64_t N, int64_t K, int64_t E, void* xp, void* stream);

/* Weighted combine: out[t] = sum_k w[t,k] y[slot_row[t*K+k]] over slots that
 * have a computed row and are not dropped (drop may be NULL); fp32 sums, one
 * write per token.  Replaces the weighted scatter of
 * pkg/distributed/moe_layer.py L:347-353 (and the masked_fill of L:305). */
int moe_combine(const void* y, int dtype, const void* w, int w_dtype, const uint8_t* drop,
                const int32_t* slot_row, const int32_t* offsets, int64_t N, int64_t K, int64_t H, int64_t E,
                void* out, void* stream);

/* Combine backward: dy[row] = w'[t,k] dout[t]; dw[t,k] = <dout[t], y[row]>
 * (0 for dropped slots and slots without a computed row).  The autograd
 * backward of L:347-353 in the reference. */
int moe_combine_bwd(const void* dout, const void* y, int dtype, const void* w, int w_dtype, const uint8_t* drop,
                    const int32_t* slot_row, const int32_t* offsets, int64_t N, int64_t K, int64_t H, int64_t E,
                    void* dy, void* dw, void* stream);

/* Permute backward: dx[t] = addend[t] (NULL = 0) + sum_k dxp[slot_row[t*K+k]]
 * over computed rows.  The autograd backward of L:318-319. */
int moe_unpermute_sum(const void* dxp, const void* addend, int dtype, const int32_t* slot_row,
                      const int32_t* offsets, int64_t N, int64_t K, int64_t H, int64_t E, void* dx, void* stream);

/* ------------------------------------------------------------------------
 * SwiGLU expert grouped GEMM, bf16 (fp32 accumulate).  For the rows of each
 * expert segment:  act = silu(xp Wg_e^T) * (xp Wu_e^T),  y = act Wd_e^T,
 * with w_gate / w_up [E, F, H] and w_down [E, H, F] (the reference's
 * nn.Linear [out, in] layout per expert).  hgu [R, 2F] keeps the two
 * pre-activations [g | u] for the backward; it may be NULL when no backward
 * follows (inference: the forward then stores only act and y; also for
 * moe_swiglu_fwd_fp8).  Replaces the expert loop of
 * pkg/distributed/moe_layer.py L:326-337 over _SwiGLUExpert.forward
 * (L:197-198; F.linear at tp=1, pkg/distributed/tensor_parallel.py
 * L:117-121, L:195-199).
 *
 * Backward: dh [R, 2F] = [dg | du], dxp [R, H], and the weight gradients
 * dw_gate / dw_up [E, F, H], dw_down [E, H, F] (experts without rows get 0).
 * Limits: H % 8 == 0, F % 32 == 0, E <= 1024.
 * ---------------------------------------------------------------------- */
size_t moe_swiglu_workspace(int64_t E);
int moe_swiglu_fwd(const void* xp, const void* w_gate, const void* w_up, const void* w_down,
                   const int32_t* offsets, int64_t R, int64_t H, int64_t F, int64_t E,
                   void* act, void* hgu, void* y, void* workspace, size_t ws_bytes, void* stream);
int moe_swiglu_bwd(const void* dy, const void* xp, const void* act, const void* hgu, const void* w_gate,
                   const void* w_up, const void* w_down, const int32_t* offsets, int64_t R, int64_t H,
                   int64_t F, int64_t E, void* dh, void* dxp, void* dw_gate, void* dw_up, void* dw_down,
                   void* workspace, size_t ws_bytes, void* stream);

/* The same grouped SwiGLU products in float32 (the reference module's default dtype): every tensor fp32,
 * v_mfma_f32_32x32x2_f32 (fp32 products and sums, as the reference's float32 F.linear experts compute them,
 * moe_layer.py L:166-198, L:326-337).  Limits: H % 4 == 0, F % 32 == 0, E <= 1024; the operands 16-byte
 * aligned.  Workspace: moe_swiglu_f32_workspace(E) bytes. */
size_t moe_swiglu_f32_workspace(int64_t E);
int moe_swiglu_fwd_f32(const float* xp, const float* w_gate, const float* w_up, const float* w_down,
                       const int32_t* offsets, int64_t R, int64_t H, int64_t F, int64_t E,
                       float* act, float* hgu, float* y, void* workspace, size_t ws_bytes, void* stream);
int moe_swiglu_bwd_f32(const float* dy, const float* xp, const float* act, const float* hgu, const float* w_gate,
                       const float* w_up, const float* w_down, const int32_t* offsets, int64_t R, int64_t H,
                       int64_t F, int64_t E, float* dh, float* dxp, float* dw_gate, float* dw_up, float* dw_down,
                       void* workspace, size_t ws_bytes, void* stream);

/* ----------------------------------------------------------------------
 * fp8 (e4m3, OCP) forward of the expert FFN: a variant of moe_permute +
 * moe_swiglu_fwd (moe_layer.py L:317-319 and the expert loop L:166-198,
 * L:326-337) with half the dispatch bytes and the gfx950 fp8 MFMA.  Every
 * quantized row carries one fp32 scale = absmax(row) / 448 (1 for a zero
 * row); elements are x * (448 / absmax) in fp32 (1 for a zero row) rounded
 * to nearest even.  The reference has
 * no fp8 path: its results are the bf16 path's up to this quantization.
 *
 * moe_quant_rows_fp8: src [rows, ld] (MOE_BF16 / MOE_F32, first `cols`
 * columns) -> dst [rows, cols] e4m3 bytes, scale [rows] f32.  cols % 16 == 0.
 * moe_permute_fp8: the quantized dispatch payload: row slot_row[t*K+k] of
 * xq [N*K, H] is token t of x quantized, sx its scale (rows the plan leaves
 * empty, or past offsets[E], are not written).
 * moe_swiglu_fwd_fp8: act, hgu, y as moe_swiglu_fwd (bf16) from xq / sx and
 * the quantized weights wg_q, wu_q [E, F, H], wd_q [E, H, F] with scales
 * sg, su [E, F], sd [E, H] (moe_quant_rows_fp8 over the weight rows).  The
 * gate/up epilogue writes act block-quantized into the workspace for the
 * down projection (OCP MX: every 32 consecutive elements of a row share a
 * power-of-two scale 2^e, e the smallest integer with absmax <= 448 * 2^e,
 * stored as the E8M0 byte e + 127; elements x * 2^-e rounded to nearest
 * even).  Workspace layout after the moe_swiglu_workspace(E) tile tables:
 * act e4m3 [R, F], then at the next 256-byte boundary the scale bytes
 * [F / 128][R rounded up to 4][4].  act and hgu may be NULL (inference).
 * H % 16 == 0, F % 32 == 0.
 * ---------------------------------------------------------------------- */
int moe_quant_rows_fp8(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld, void* dst,
                       float* scale, void* stream);
int moe_permute_fp8(const void* x, int x_dtype, const int32_t* slot_row, const int32_t* offsets, int64_t N,
                    int64_t K, int64_t E, int64_t H, void* xq, float* sx, void* stream);
size_t moe_swiglu_fwd_fp8_workspace(int64_t R, int64_t F, int64_t E);
int moe_swiglu_fwd_fp8(const void* xq, const float* sx, const void* wg_q, const float* sg, const void* wu_q,
                       const float* su, const void* wd_q, const float* sd, const int32_t* offsets, int64_t R,
                       int64_t H, int64_t F, int64_t E, void* act, void* hgu, void* y, void* workspace,
                       size_t ws_bytes, void* stream);

/* ----------------------------------------------------------------------
 * RMSNorm in front of the router (the caller step before the routed path):
 * replaces RMSNorm.forward (moe-engine/pkg/models/moe.py L:83-86) as used by
 * ToyMoEBlock.forward (L:125-126, x + moe(norm(x))):
 *   xn = ((x * rsqrt(mean_h(x^2) + eps)) * gamma).to(x.dtype), fp32 arithmetic;
 * rstd_out [N] f32 keeps rsqrt(mean_h(x^2) + eps) for the backward.
 * x / xn dtype MOE_F32 or MOE_BF16, gamma MOE_F32 or MOE_BF16; 8 <= H <= 8192,
 * H % 8 == 0; x, gamma, xn 16-byte aligned.
 *
 * moe_rmsnorm_router_fwd: the norm with the router forward of moe_router_fwd
 * applied to xn (same outputs, statistics, workspace contract and first-word
 * completion counter).  For bf16 x and gate with E <= 16 one kernel reads x
 * from HBM once, producing xn and the routing; otherwise the norm kernel runs
 * first and the router kernels read xn.
 *
 * moe_rmsnorm_bwd: dx = rstd (g - xhat mean_h(g xhat)), xhat = x rstd,
 * g = gamma * u, u = dxn + dxn2 (dxn2 optional: a second gradient of xn, e.g.
 * the router's; the sum is rounded to x's dtype, as a sum of two gradients of
 * xn is); dgamma = sum_t u xhat in gamma's dtype, summed in a fixed order
 * (deterministic).
 *
 * moe_rmsnorm_router_bwd: the backward of moe_rmsnorm_router_fwd: the router
 * backward of moe_router_bwd over xn (same grad_w / grad_aux / grad_z / cnt
 * contract; dwg_out in wg's dtype) and the norm backward of dxn plus the
 * router's gradient of xn (dxn may be null: no gradient from the expert path).
 * For bf16 x and gate with E <= 16 and H % 256 == 0 the router's gradient of
 * xn is formed inside the norm kernel from dL/dlogits and never reaches HBM;
 * otherwise moe_router_bwd writes it to the workspace and moe_rmsnorm_bwd
 * adds it.
 * ---------------------------------------------------------------------- */
int moe_rmsnorm_fwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype, float eps, int64_t N,
                    int64_t H, void* xn_out, float* rstd_out, void* stream);
size_t moe_rmsnorm_router_fwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype, int wg_dtype);
int moe_rmsnorm_router_fwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype, float eps,
                           const void* wg, int wg_dtype, const float* bias, int64_t N, int64_t H, int64_t E,
                           int64_t K, void* xn_out, float* rstd_out, int64_t* idx_out, void* w_out, int w_dtype,
                           float* logits_out, float* lse_out, int64_t* cnt_out, float* stats_out, float aux_coef,
                           float z_coef, float* aux_out, float* z_out, void* workspace, size_t ws_bytes,
                           void* stream);
size_t moe_rmsnorm_bwd_workspace(int64_t N, int64_t H);
int moe_rmsnorm_bwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype, const float* rstd,
                    const void* dxn, const void* dxn2, int64_t N, int64_t H, void* dx_out, void* dgamma_out,
                    void* workspace, size_t ws_bytes, void* stream);
size_t moe_rmsnorm_router_bwd_workspace(int64_t N, int64_t H, int64_t E, int64_t K, int x_dtype, int wg_dtype);
int moe_rmsnorm_router_bwd(const void* x, int x_dtype, const void* gamma, int gamma_dtype, const float* rstd,
                           const void* xn, const void* wg, int wg_dtype, const float* logits, const int64_t* idx,
                           const void* grad_w, int gw_dtype, const int64_t* cnt, const float* grad_aux,
                           const float* grad_z, float aux_coef, float z_coef, const void* dxn, int64_t N, int64_t H,
                           int64_t E, int64_t K, void* dx_out, void* dgamma_out, void* dwg_out, void* workspace,
                           size_t ws_bytes, void* stream);

/* ----------------------------------------------------------------------
 * Per-step routing telemetry on the device: replaces the host-side routing
 * block of the reference's train step (moe-engine/train.py L:360-399, which
 * reads the RouterProfile of moe_router.py L:594-612 / L:690-745 and the
 * dispatch counts with .item() synchronisations every step).
 *
 * moe_telemetry_record appends one record of moe_telemetry_fields() floats (16) to a ring buffer in device
 * memory from the router's stats vector (stats_out of moe_router_fwd / moe_rmsnorm_router_fwd, same stream)
 * and, optionally, the planner's drop count (ndrop of moe_plan; null = no capacity drops):
 *   [0] step (int32 bits: `step`, or the record's ordinal when step < 0)
 *   [1] load imbalance  [2] z statistic  [3] tokens/expert mean
 *   [4] tokens/expert std  [5] dead experts  [6] active experts
 *   [7] routing efficiency = dispatched / (capacity_factor * N * K)
 *   [8] dropped fraction = ndrop / (N * K)  [9] aux statistic
 *   [10] non-finite logits  [11] dispatched slots  [12..15] zero
 * ring: capacity * 16 floats of records followed by one int32 write cursor (the number of records appended
 * so far; zero it once before the first record).  Record n goes to slot n % capacity; the kernel advances
 * the cursor with an atomic add, so a launch captured in a HIP graph appends a new record on every replay.
 * No host synchronisation; the caller copies the ring (cursor included) when it logs.
 * ---------------------------------------------------------------------- */
int moe_telemetry_fields(void);
int moe_telemetry_record(const float* stats, int64_t E, int64_t N, int64_t K, float capacity_factor,
                         const int32_t* ndrop, int64_t step, float* ring, int64_t capacity, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355_H */
