/*
 * resihp_moe.h -- C ABI of the MI355X (gfx950) MoE expert-parallel layer hot path.
 *
 * Every entry point takes raw device pointers, element counts, dtype codes and
 * a HIP stream, enqueues its kernels on that stream and returns 0 on success.
 * On failure it returns a nonzero status, enqueues nothing, and
 * rhp_last_error() returns a message for the calling thread.  The library
 * never allocates or frees device memory: callers pass outputs and workspace.
 * It keeps no state between calls, so calls are re-entrant; calls that write
 * the same buffers must be ordered by the caller's stream.
 *
 * Reference interfaces replaced (Sullivan-24/ResiHP-Megatron):
 *   route                  resihp/runtime/moe.py:75-79
 *   bincount / dispatch    resihp/runtime/moe.py:94, 97, 192-207
 *   gather                 resihp/runtime/moe.py:99, 212  (x[rows], x.index_select)
 *   expert FFN             resihp/runtime/moe.py:82-83, 96-100, 213-223
 *   combine + residual     resihp/runtime/moe.py:100-101, 225-226
 *   backward               torch autograd of the above (moe.py:116; _AllToAll.backward :164-167)
 *   expert-bias update     resihp/runtime/moe.py:64-66, 236-240
 *
 * Row layout: tokens are rows of a [T, h] row-major matrix.  Routed pairs are
 * (token t, slot j) with flat index p = t*k + j.  A dispatch plan assigns every
 * local pair a row r of the expert-contiguous ("permuted") buffers; the rows
 * of local expert i are [offsets[i], offsets[i+1]).
 */
#ifndef RESIHP_MOE_H
#define RESIHP_MOE_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RHP_ABI_VERSION 1
#define RHP_MAX_GROUPS_PER_LAUNCH 64

/* Element types. */
enum { RHP_F64 = 0, RHP_F32 = 1, RHP_BF16 = 2, RHP_E4M3 = 3, RHP_E5M2 = 4 };
/* Router scoring. */
enum { RHP_SCORE_SOFTMAX = 0, RHP_SCORE_SIGMOID = 1 };
/* Expert activation. */
enum { RHP_ACT_GELU = 0, RHP_ACT_SWIGLU = 1 };

int rhp_abi_version(void);

/* Message of the last failing call on the calling thread ("" if none). */
const char* rhp_last_error(void);

/* ------------------------------------------------------------------ routing */

/*
 * Router logits, top-k selection and gates for T tokens.
 * Replaces route() (resihp/runtime/moe.py:75-79):
 *   logits = x @ router_w^T          x: [T,h] x_dtype (F64/F32/BF16)
 *                                   router_w: [E,h] r_dtype (F64 iff x is F64, else F32)
 *   topi   = top-k of (score(logits) + bias), descending, ties to the lowest id
 *   gates  = softmax over the selected unbiased logits (score = SOFTMAX), or the
 *            selected sigmoid scores, divided by their sum if normalize (SIGMOID),
 *            times scale
 * bias ([E], r_dtype) may be NULL.  Outputs: logits [T,E] r_dtype, topi [T,k]
 * int32, gates [T,k] r_dtype.  The logits follow a fixed evaluation order
 * (segments of min(256,h) elements, each one fused-multiply-add chain, summed
 * left to right) so that results are reproducible bit for bit.
 * Requires h % 8 == 0, h % min(256,h) == 0, 1 <= k <= min(E, 16), E <= 1024.
 */
int rhp_route(const void* x, int x_dtype, const void* router_w, int r_dtype, const void* bias, int64_t T,
              int h, int E, int k, int score, int normalize, double scale, void* logits, int32_t* topi,
              void* gates, hipStream_t stream);

/* Workspace bytes rhp_dispatch needs for these sizes. */
size_t rhp_dispatch_workspace_bytes(int64_t T, int k, int E, int n_src);

/*
 * Dispatch plan of the local experts [e0, e1).
 * Replaces bincount (moe.py:94, 192) and the dispatch ordering (moe.py:97,
 * 193-207 with one device: pairs sorted stably by expert, then by p).
 *   counts[E+1]        pairs per expert for all E experts; counts[E] = ids outside [0,E)
 *   offsets[L+1]       exclusive prefix of counts[e0..e1), L = e1 - e0
 *   src_counts[n_src*L] local pairs per (source, local expert); the T tokens are
 *                      split into n_src contiguous sources by even_split
 *                      (resihp/utils/intervals.py:17-30)
 *   perm[T*k]          perm[r] = p for local rows r < offsets[L]; the rest is untouched
 *   pair_row[T*k]      row of pair p, or -1 if its expert is not local
 * Bit-exact with any stable counting sort.  Requires 1 <= L <= 1024, E <= 1024.
 */
int rhp_dispatch(const int32_t* topi, int64_t T, int k, int E, int e0, int e1, int n_src, int32_t* counts,
                 int32_t* offsets, int32_t* src_counts, int32_t* perm, int32_t* pair_row, void* workspace,
                 size_t workspace_bytes, hipStream_t stream);

/*
 * rhp_dispatch without a workspace argument and without allocating: the same
 * plan, bit for bit, with a fixed 4 MiB device array of the library (one per
 * GPU, kept until the process ends) as its workspace.  No counterpart in the
 * reference: an entry point for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Sizes whose rhp_dispatch_workspace_bytes() exceeds 4 MiB are
 * rejected.  The stream's device must be current.  All calls on one GPU share
 * its array, so calls that overlap on one GPU (different streams without
 * ordering) race; stream-ordered calls are safe, since every call writes each
 * scratch entry it reads.
 */
int rhp_dispatch_noalloc(const int32_t* topi, int64_t T, int k, int E, int e0, int e1, int n_src, int32_t* counts,
                         int32_t* offsets, int32_t* src_counts, int32_t* perm, int32_t* pair_row, hipStream_t stream);

/*
 * Aux-loss-free bias update: bias[e] += rate * sign(mean(counts) - counts[e]).
 * Replaces update_expert_bias (moe.py:64-66).  bias: [E] r_dtype; counts: int32 [E].
 */
int rhp_update_expert_bias(void* bias, int r_dtype, const int32_t* counts, int E, double rate,
                           hipStream_t stream);

/* ---------------------------------------------------------- permute/combine */

/*
 * Permute tokens into expert-contiguous rows: xp[pair_row[t*k+j]] = x[t] for
 * every local pair.  Replaces x.index_select(0, idx_i) (moe.py:212) / x[rows]
 * (moe.py:99).  Each token row is read once and written to its k rows.
 * dtype: F64 / F32 / BF16.
 */
int rhp_permute(const void* x, int dtype, int64_t T, int h, int k, const int32_t* pair_row, void* xp,
                hipStream_t stream);

/*
 * Weighted unpermute + residual:
 *   out[t] = x[t] + sum over local slots j, in ascending expert id, of gates[t,j] * y[pair_row[t*k+j]]
 *            + sum_s shared_y[s][t]
 * Replaces zeros.index_add(0, idx_i, gates[idx_i,idx_j] * back) and x + combined
 * (moe.py:225-226; moe.py:100-101).  topi gives the ascending-id order.
 * y, x, out, shared_y: dtype (F64/F32/BF16); gates: g_dtype (F64/F32).
 * shared_y is a host array of n_shared (<= 8) device pointers; may be NULL if 0.
 */
int rhp_combine(const void* y, const void* x, const void* gates, int g_dtype, const int32_t* topi,
                const int32_t* pair_row, const void* const* shared_y, int n_shared, int dtype, int64_t T, int h,
                int k, void* out, hipStream_t stream);

/*
 * Backward of the weighted unpermute:
 *   dy[pair_row[t*k+j]] = gates[t,j] * dout[t]
 *   dgates[t,j]         = <dout[t], y[pair_row[t*k+j]]>   (0 for non-local slots)
 * dgates has g_dtype.
 */
int rhp_combine_bwd(const void* dout, const void* y, const void* gates, int g_dtype, const int32_t* pair_row,
                    int dtype, int64_t T, int h, int k, void* dy, void* dgates, hipStream_t stream);

/*
 * Router backward to the selected logits: dlogits_sel[t,j] = d loss / d logits[t, topi[t,j]]
 * given dgates [T,k], the gates and logits of rhp_route (r_dtype), for the
 * same score / normalize / scale.  Logits of unselected experts get no gradient
 * (the selection is piecewise constant).
 */
int rhp_route_bwd(const void* dgates, const void* gates, const void* logits, const int32_t* topi, int r_dtype,
                  int64_t T, int E, int k, int score, int normalize, double scale, void* dlogits_sel,
                  hipStream_t stream);

/*
 * Token-side backward:
 *   dx[t] = dout[t] + sum_j dxp[pair_row[t*k+j]] + sum_j dlogits_sel[t,j] * router_w[topi[t,j]]
 *           + sum_s shared_dx[s][t]
 * (residual + scatter-add of the permuted input gradient + router input gradient).
 * dout, dxp, dx, shared_dx: dtype; dlogits_sel, router_w: r_dtype.
 */
int rhp_token_bwd(const void* dout, const void* dxp, const int32_t* pair_row, const void* dlogits_sel,
                  const int32_t* topi, const void* router_w, int r_dtype, const void* const* shared_dx, int n_shared,
                  int dtype, int64_t T, int h, int E, int k, void* dx, hipStream_t stream);

/* Workspace bytes rhp_router_wgrad needs. */
size_t rhp_router_wgrad_workspace_bytes(int64_t T, int h, int E, int k, int r_dtype);

/*
 * Router weight gradient dW[e,:] = sum over pairs p = t*k+j routed to e of
 * dlogits_sel[p] * x[t,:].  perm / offsets are a dispatch plan over ALL E
 * experts (e0 = 0, e1 = E); each expert's rows are summed in plan order in
 * pieces of 64 rows, and the pieces are added in ascending order, so the
 * result is deterministic.  Accumulation in r_dtype.  dw: [E,h] r_dtype.
 */
int rhp_router_wgrad(const void* dlogits_sel, const int32_t* perm, const int32_t* offsets, const void* x,
                     int x_dtype, int r_dtype, int64_t T, int h, int E, int k, void* dw, void* workspace,
                     size_t workspace_bytes, hipStream_t stream);

/* ----------------------------------------- sending side of expert parallelism */

/*
 * Send plan of one source: EPRuntime.forward (resihp/runtime/moe.py:189-211)
 * up to the exchange.  The pairs of expert e, in (token, slot) order, go to
 * e's holders in the EP group by smooth_weighted_round_robin
 * (resihp/plan/expert_placement.py:150-164, moe.py:193-198); the send order is
 * device-major (the group's devices in world order), then expert-major, then
 * (token, slot) ascending (moe.py:199-207).
 *   topi [T*k], counts [E+1], offsets [E+1], pair_row [T*k]: the plan of
 *       rhp_dispatch with the window [0, E) (every expert), same topi
 *   pick_off [E+1], pick_dev [pick_off[E]], pick_rank [pick_off[E]],
 *   period_cnt [E*n_dev]: one period of every expert's holder picks (a smooth
 *       weighted round robin repeats after the sum of its weights): position
 *       r of expert e's period sends to device pick_dev[pick_off[e] + r]
 *       (0 <= d < n_dev), as that device's pick_rank-th pick of the period;
 *       period_cnt[e * n_dev + d] = picks of d in the period.  Built on the
 *       host from the placement (placement.send_tables).
 * Outputs (int32, device):
 *   send_counts [n_dev * E]   counts[d, e] of moe.py:199-207 (their row sums are the
 *                             split sizes of moe.py:210)
 *   send_offsets [n_dev*E+1]  exclusive prefix of send_counts in send order; the rows
 *                             for device d are [send_offsets[d*E], send_offsets[(d+1)*E])
 *   send_perm [T*k]           send row -> flat pair t*k + j (rows < send_offsets[n_dev*E];
 *                             idx_i = pair / k, idx_j = pair % k of moe.py:208-209)
 *   send_row [T*k]            pair -> send row, -1 for an expert id outside [0, E)
 * rhp_permute and rhp_combine with send_row as pair_row build the send buffer
 * (x.index_select(0, idx_i), moe.py:212) and combine the returned rows
 * (moe.py:225-226).  n_dev * E <= 65536.  Bit-exact with the reference order.
 */
int rhp_ep_send_plan(const int32_t* topi, int64_t T, int k, int E, int n_dev, const int32_t* counts,
                     const int32_t* offsets, const int32_t* pair_row, const int32_t* pick_off, const int32_t* pick_dev,
                     const int32_t* pick_rank, const int32_t* period_cnt, int32_t* send_counts,
                     int32_t* send_offsets, int32_t* send_perm, int32_t* send_row, hipStream_t stream);

/* ----------------------------------------- received rows (receiving side of expert parallelism) */

/*
 * Plan of a received buffer: the receiving side of EPRuntime.forward
 * (resihp/runtime/moe.py:199-226).  Each source sends its rows for this GPU
 * expert-major, (token, slot) ascending within an expert (moe.py:199-207), and
 * the all-to-all concatenates the sources (:209-212), so the received buffer
 * holds chunk (s, e) of recv_counts[s * L + e] rows, source-major; the
 * reference runs the expert FFN chunk by chunk in that order (:213-223).  The
 * grouped GEMMs need each local expert's rows together:
 *   offsets[L+1]       expert-major group offsets (sources in order within an expert)
 *   sort_row[rows]     expert-major row r holds received row sort_row[r]
 *   unsort_row[rows]   received row q is expert-major row unsort_row[q]
 * recv_counts: [n_src, L] int32 on the device, the local experts' columns of the
 * exchanged counts (moe.py:209); rows must equal their sum (the reference
 * materialises the split sizes on the host, moe.py:210-211), which the kernel
 * writes to offsets[L].  If they differ, every map entry without a partner
 * among the first `rows` rows is -1 (the products read such a row as zeros and
 * drop its stores).  n_src * L <= 8192.
 */
int rhp_recv_plan(const int32_t* recv_counts, int n_src, int L, int64_t rows, int32_t* offsets, int32_t* sort_row,
                  int32_t* unsort_row, hipStream_t stream);

/*
 * Row gather: dst[r] = src[idx[r]] for r < rows (whole rows of h elements,
 * dtype F64 / F32 / BF16, 16-byte aligned); an index outside [0, src_rows)
 * gives a zero row.  With sort_row it regroups received rows expert-major;
 * with unsort_row it puts expert outputs and input gradients back into the
 * received order, in which they return to their sources (moe.py:224).
 */
int rhp_gather_rows(const void* src, int dtype, int64_t src_rows, int h, const int32_t* idx, int64_t rows,
                    void* dst, hipStream_t stream);

/* ------------------------------------------------------- expert grouped GEMMs */

/*
 * The four grouped expert GEMMs of a SwiGLU or GELU FFN (moe.py:82-83 applied
 * to every local expert at once; moe.py:96-100, 213-223).  Group g (a local
 * expert) owns M_g = offsets[g+1] - offsets[g] rows.  Row buffers are passed
 * as host arrays of G device pointers; with rows_from_offsets = 1 group g's
 * rows start at row offsets[g] of its buffer (routed experts: every entry is
 * the same permuted buffer), with 0 at row 0 (shared experts: one buffer per
 * group).  offsets is a device array of G+1 int32.  rows_cap bounds the
 * launch: with rows_from_offsets = 1 the shared buffer holds rows_cap >=
 * offsets[G] rows; with rows_from_offsets = 0 every group's buffer holds
 * rows_cap rows and no group has more (offsets[g+1] - offsets[g] <= rows_cap).
 * Rows past rows_cap are never read or written.  Weights are per-group
 * device pointers, so each expert keeps its own parameter tensor.
 *
 *   fc1 weight w1[g]: [F1, h] row-major, F1 = 2f (SwiGLU: gate rows, then up rows) or f (GELU)
 *   fc2 weight w2[g]: [h, f]
 *
 * dtype: BF16, F32 or F64.  bfloat16 products with h % 64 == 0, f % 64 == 0
 * and weights below 2 GiB run on the MFMA kernel, for any number of rows; its
 * operand pointers must then be 16-byte aligned (an unaligned pointer is an
 * error).  Every other call runs the generic kernel (float32 / float64, or
 * bfloat16 shapes the MFMA kernel does not take); rhp_expert_gemm_kernel()
 * says which one a call takes.  Groups beyond RHP_MAX_GROUPS_PER_LAUNCH are
 * split into several launches.
 */

/* Which kernel the expert GEMM entry points run for these operands: the MFMA kernel or the generic one. */
enum { RHP_GEMM_KERNEL_GENERIC = 0, RHP_GEMM_KERNEL_MFMA = 1 };
int rhp_expert_gemm_kernel(int dtype, int act, int h, int f);

/*
 * K-split workspace of the row-grouped products (forward and input-gradient;
 * optional, NULL disables the split).  On each XCD the tiles past the last
 * whole round of one tile per CU are cut along K into pieces that run on the
 * otherwise idle CUs; pieces keep fp32 partial tiles here and the last piece
 * of a tile to finish adds them in piece order (deterministic) and writes the
 * tile.  The workspace ends in arrival counters that must be zero before its
 * first use; every call that completes leaves them zero again.  Calls that
 * share a workspace must not run concurrently (stream-order them, or give
 * each stream its own workspace).  No reference counterpart: scheduling
 * only, the products are those of moe.py:82-83.
 */
size_t rhp_expert_split_workspace_bytes(void);

/* Zeroes the arrival counters of a K-split workspace (a fill kernel on the
 * stream): before its first use, and after a call that did not complete. */
int rhp_expert_split_workspace_reset(void* split_ws, size_t split_ws_bytes, hipStream_t stream);

/*
 * h = xp[r] @ w1^T  ([M_g, F1]);  act[r] = silu(gate) * up  or  gelu(h)  ([M_g, f]);
 * hpre[r] = what the backward of the activation needs: for SwiGLU the two
 * factors of the activation gradient, [up * silu'(gate) | silu(gate)]
 * ([M_g, 2f], gate = h[:, :f], up = h[:, f:]; the forward has the sigmoid at
 * hand, and the backward then costs two products per element); for GELU the
 * pre-activation h itself.
 */
int rhp_expert_fc1_fwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype, int act,
                       int h, int f, const void* const* xp, const void* const* w1, void* const* hpre,
                       void* const* act_out, void* split_ws, size_t split_ws_bytes, hipStream_t stream);

/* y[r] = act[r] @ w2^T  ([M_g, h]). */
int rhp_expert_fc2_fwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype, int h,
                       int f, const void* const* act_in, const void* const* w2, void* const* y, void* split_ws,
                       size_t split_ws_bytes, hipStream_t stream);

/*
 * Backward through fc2 and the activation:
 *   dact = dy @ w2;  dhpre = activation backward of dact from hpre  ([M_g, F1]):
 *   SwiGLU [dact * hpre[:, :f] | dact * hpre[:, f:]], GELU dact * gelu'(hpre)
 *   dw2[g] = dy_g^T @ act_g  ([h, f])      (written, not accumulated)
 * dhpre may be NULL to skip the input-gradient product (then hpre and w2 are
 * not read), or dw2 NULL to skip the weight gradient, not both.  The two
 * products are independent, so a caller may run them on two streams.
 */
int rhp_expert_fc2_bwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype, int act,
                       int h, int f, const void* const* dy, const void* const* act_in, const void* const* hpre,
                       const void* const* w2, void* const* dhpre, void* const* dw2, void* split_ws,
                       size_t split_ws_bytes, hipStream_t stream);

/*
 * Backward through fc1:
 *   dxp = dhpre @ w1  ([M_g, h]);   dw1[g] = dhpre_g^T @ xp_g  ([F1, h])   (written, not accumulated)
 * dxp may be NULL to skip the input gradient, or dw1 NULL to skip the weight
 * gradient, not both; the two products may run on two streams.
 */
int rhp_expert_fc1_bwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype, int act,
                       int h, int f, const void* const* dhpre, const void* const* xp, const void* const* w1,
                       void* const* dxp, void* const* dw1, void* split_ws, size_t split_ws_bytes,
                       hipStream_t stream);

/*
 * The same products on received rows (moe.py:213-226): the expert FFN of the
 * rows a GPU received from its sources, which arrive source-major, (src, e)
 * chunks (moe.py:211-212), and return in the same order (moe.py:224).  With
 * the rhp_recv_plan maps, expert-major row r (the grouped order of offsets)
 * is received row sort_row[r]; the products below read or write received rows
 * directly through such a map, so no regrouped copy is made:
 *   fc1_fwd_gather:    row r of the grouped product reads src[src_idx[r]]
 *   fc2_fwd_scatter:   y[y_idx[r]] = act[r] @ w2^T (rows of y no index names are not written)
 *   fc2_dgrad_gather:  the input-gradient product of rhp_expert_fc2_bwd on dy[dy_idx[r]]
 *   fc1_dgrad_scatter: dx[dx_idx[r]] = dhpre[r] @ w1
 * Index arrays hold rows_cap int32 entries (rows_cap >= offsets[G]); an index
 * outside [0, src_rows) reads a zero row, one outside [0, y_rows) drops the
 * row.  Grouped-order operands (hpre, act, dhpre) are single buffers of
 * rows_cap rows.  The results equal those of rhp_gather_rows followed by the
 * plain product, bit for bit.  On the MFMA kernel a mapped buffer must be
 * 16-byte aligned and hold fewer than 2^31 / (2 ld) - 1 rows (ld = h), which
 * is an error otherwise.  No reference counterpart as entry points: they fuse
 * the regrouping gathers of moe.py:213-226 into the products.
 */
int rhp_expert_fc1_fwd_gather(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h, int f,
                              const void* src, int64_t src_rows, const int32_t* src_idx, const void* const* w1,
                              void* hpre, void* act_out, void* split_ws, size_t split_ws_bytes, hipStream_t stream);
int rhp_expert_fc2_fwd_scatter(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int h, int f,
                               const void* act_in, const void* const* w2, void* y, int64_t y_rows,
                               const int32_t* y_idx, void* split_ws, size_t split_ws_bytes, hipStream_t stream);
int rhp_expert_fc2_dgrad_gather(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h, int f,
                                const void* dy, int64_t dy_rows, const int32_t* dy_idx, const void* hpre,
                                const void* const* w2, void* dhpre, void* split_ws, size_t split_ws_bytes,
                                hipStream_t stream);
int rhp_expert_fc1_dgrad_scatter(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h, int f,
                                 const void* dhpre, const void* const* w1, void* dx, int64_t dx_rows,
                                 const int32_t* dx_idx, void* split_ws, size_t split_ws_bytes, hipStream_t stream);

/*
 * fc1's input-gradient product with the router's term of the token backward
 * folded into its epilogue: for expert-major row r of group g (expert e0 + g),
 *   dxp[r] = dhpre[r] @ w1 + dlogits_sel[perm[r]] * router_w[e0 + g]
 * rounded once to the row dtype.  rhp_token_bwd then runs without dlogits_sel:
 * sum_j dxp[row_j] holds every slot's router term (moe.py:76-79, 164-167).
 * Valid only when every expert of the layer is local (all pairs have a row);
 * with a window the router terms of other devices' pairs would be missing.
 * router_w: fp32 [E, h]; perm: the dispatch plan's row -> pair map;
 * dlogits_sel: fp32 [T, k] (rhp_route_bwd).  BF16 or F32 experts.  No reference
 * counterpart as an entry point: a fusion of two autograd terms.
 */
int rhp_expert_fc1_dgrad_router(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h, int f,
                                const void* const* dhpre, const void* const* w1, const float* router_w, int e0,
                                const int32_t* perm, const float* dlogits_sel, void* const* dxp, void* split_ws,
                                size_t split_ws_bytes, hipStream_t stream);

/* ------------------------------------------------------------------ optimizer step */

/*
 * One Adam step over `count` tensors of one dtype (F64, F32 or BF16), in
 * place: resihp/runtime/optim.py:32-46 (the update of
 * torch.optim.Adam(foreach=False); moment state exp_avg / exp_avg_sq of the
 * parameter's dtype, as optim.py:24-25 allocates it).  params, exp_avg,
 * exp_avg_sq and numel are host arrays of `count` entries; grads may be NULL
 * or hold NULL entries (a parameter without a gradient steps with a zero
 * gradient, optim.py:38).  `step` is the step number after this update
 * (optim.py:33: step_count += 1 first), from 1.  Each element evaluates the
 * operations of optim.py:39-46 in order with their torch roundings, IEEE
 * square root and division; bfloat16 tensors round every intermediate to
 * bfloat16 and the weight decay to bfloat16 (torch's add(alpha=)).  All
 * tensors must be 16-byte aligned.  One pass over the data: 14 bytes per
 * bfloat16 element (7 per array element read or written once).
 */
int rhp_adam_step(int count, void* const* params, const void* const* grads, void* const* exp_avg,
                  void* const* exp_avg_sq, const int64_t* numel, int dtype, double lr, double beta1, double beta2,
                  double eps, double weight_decay, int64_t step, hipStream_t stream);

/* ------------------------------------------------------------------ fp8 experts (delayed scaling) */

/*
 * FP8 expert GEMMs with per-tensor delayed scaling.  The reference keeps an
 * FP8-style amax history per layer (resihp/runtime/reference_model.py:44-46,
 * 204-207): a buffer of hist_len entries, the iteration's amax prepended
 * newest-first when the iteration ends (:212-216).  Here every quantised
 * tensor (the expert-input rows, the SwiGLU output rows, their gradients and
 * each expert weight) has such a history (float32 [hist_len]) and a pending
 * amax (uint32 holding float bits, reset to 0 by the roll).
 *
 * Scale of a cast: fp8_max / max(history) / 2^margin (1 if that maximum is not
 * a positive finite number); q = fp8(clamp(x * scale, -fp8_max, fp8_max)),
 * round to nearest even, OCP e4m3 (max 448) or e5m2 (max 57344).
 */

/* poff[g+1] = poff[g] + roundup(offsets[g+1] - offsets[g], align); align a multiple of 128. */
int rhp_fp8_padded_offsets(const int32_t* offsets, int G, int align, int32_t* poff, hipStream_t stream);

/*
 * Cast bf16 rows to fp8 (fmt RHP_E4M3 or RHP_E5M2) with the scale of `history`:
 *   x:   [rows, cols] bf16, row pitch ldx; expert g owns rows [offsets[g], offsets[g+1])
 *   q:   row-major fp8 copy [rows, cols] (row pitch cols), or NULL
 *   qt:  transposed copy per expert, [cols, R_g] at qt + cols * poff[g] with
 *        R_g = poff[g+1] - poff[g]; rows past the expert's count are zero; or NULL
 * Raises *amax_bits to max |x| over the cast rows (float bits, atomic max) and
 * writes *scale_inv = 1 / scale.  cols must be a multiple of 64; rows_cap
 * bounds offsets[G] - offsets[0].
 */
int rhp_fp8_cast(const void* x, int x_dtype, int64_t ldx, int cols, int G, const int32_t* offsets,
                 const int32_t* poff, int64_t rows_cap, const float* history, int hist_len, int fmt, int margin,
                 uint32_t* amax_bits, float* scale_inv, void* q, void* qt, hipStream_t stream);

/*
 * rhp_fp8_cast of n whole tensors in one launch (the expert weights of a
 * layer), each with its own history, amax and 1 / scale, row-major codes only:
 * x[i] bf16 [rows[i], cols[i]] contiguous, q[i] fp8 [rows[i], cols[i]].  Codes,
 * amax and 1 / scale equal those of one rhp_fp8_cast per tensor.  Host arrays
 * of n entries; cols[i] a multiple of 64.
 */
int rhp_fp8_cast_many(int n, const void* const* x, const int64_t* rows, const int64_t* cols,
                      const float* const* history, int hist_len, int fmt, int margin, uint32_t* const* amax_bits,
                      float* const* scale_inv, void* const* q, hipStream_t stream);

/*
 * rhp_permute of bf16 rows with fp8 codes as the output: q [rows, h] receives
 * the row-major codes that rhp_fp8_cast would write for the bf16 rows that
 * rhp_permute stores, with the scale of `history`; *amax_bits rises to their
 * max |value| and *scale_inv = 1 / scale, bit for bit as permute then cast
 * (T == 0 writes nothing; q must be a valid 16-byte aligned pointer even when
 * no pair is local).
 * Replaces the dispatch copy of resihp/runtime/moe.py:78 followed by the
 * input cast of the fp8 expert products (reference_model.py:188-203).
 */
int rhp_permute_fp8(const void* x, int64_t T, int h, int k, const int32_t* pair_row, int fmt,
                    const float* history, int hist_len, int margin, uint32_t* amax_bits, float* scale_inv, void* q,
                    hipStream_t stream);

/*
 * rhp_combine_bwd (bf16, float32 gates, top-k <= 8) with dy leaving as fp8
 * codes: q [rows, h] receives the codes of the bf16 dy rows, bit for bit as
 * rhp_combine_bwd then rhp_fp8_cast; dgates as rhp_combine_bwd.
 */
int rhp_combine_bwd_fp8(const void* dout, const void* y, const float* gates, const int32_t* pair_row, int64_t T,
                        int h, int k, float* dgates, int fmt, const float* history, int hist_len, int margin,
                        uint32_t* amax_bits, float* scale_inv, void* q, hipStream_t stream);

/* End of iteration for n tensors: history[i] = [amax_i, history[i][0 .. hist_len-2]], amax_i = 0 (reference_model.py:215). */
int rhp_fp8_amax_roll(float* history, uint32_t* amax_bits, int n, int hist_len, hipStream_t stream);

/*
 * Grouped fp8 product, bf16 output, with the epilogues of the bf16 entry points.
 * Replaces the expert FFN products of resihp/runtime/moe.py:82-83 and their
 * autograd backward when the experts run in fp8.  The result is multiplied by
 * y_scale_inv[0] * x_scale_inv[g * x_scale_stride].  Modes 0 and 1 read both
 * operands K-contiguous; modes 2 and 3 read x (and in mode 3 also y)
 * N-contiguous, transposing in LDS, so they take the row-major codes where
 * modes 0 and 1 need transposed copies, with the same sums bit for bit:
 *   mode 0: out[r, n] = sum_k y[g][r, k] x[g][n, k] for the rows r of expert g
 *                (offsets; y[g] holds all rows, row pitch ldy; x[g]: [N or 2f, K], pitch ldx).
 *                epi: 0 store, 1 SwiGLU forward (x rows [gate; up], out = hpre [.., 2f] as
 *                rhp_expert_fc1_fwd writes it, c2 = act,
 *                N = f), 2 GELU forward (c2 = act), 3 SwiGLU backward, 4 GELU backward
 *                (aux = hpre); K a multiple of 128.
 *   mode 1: out_g[o, n] = sum_t y_g[o, t] x_g[n, t] over the R_g padded rows of expert g,
 *                with y_g = y[0] + Mo * poff[g], x_g = x[0] + N * poff[g] (the qt copies of
 *                rhp_fp8_cast; offsets = poff), row pitch R_g; epi must be 0.
 *   mode 2: out[r, n] = sum_k y[g][r, k] x[g][k, n]: as mode 0 with each x[g] held [K, N]
 *                (row pitch ldx >= N), the input-gradient products on the row-major weight
 *                codes; epi 0, 3 or 4; y e5m2.
 *   mode 3: out_g[o, n] = sum_t y[0][t, o] x[0][t, n] over the rows t of expert g
 *                (offsets[g] .. offsets[g+1], not padded): the weight gradients on the row-major
 *                codes (y pitch ldy >= Mo, x pitch ldx >= N); epi 0; y e5m2.
 * y_fmt is the format of y, x_fmt of x (RHP_E4M3 / RHP_E5M2); x must be e4m3.
 * Outputs c[g] (and c2[g]) are bf16 with row pitches ldc (ldc2).
 */
int rhp_fp8_gemm(int mode, int epi, int G, const int32_t* offsets, int64_t rows_cap, int y_fmt, int x_fmt, int N,
                 int K, int Mo, int f, const void* const* y, int64_t ldy, const void* const* x, int64_t ldx,
                 void* const* c, int64_t ldc, void* const* c2, int64_t ldc2, const void* const* aux, int64_t ldaux,
                 const float* y_scale_inv, const float* x_scale_inv, int x_scale_stride, hipStream_t stream);

/*
 * A row-grouped rhp_fp8_gemm (mode 0, or mode 2 with x_kn = 1) whose epilogue casts its bf16
 * activation output straight to fp8, fusing the cast that the next products
 * need (the quantise step of the fp8 recipe, reference_model.py:204-207, on
 * the expert FFN of moe.py:82-83 and its backward):
 *   epi 1 / 2 (SwiGLU / GELU forward): c = hpre (bf16, as rhp_fp8_gemm); the
 *            activation [rows, N] is cast instead of stored (no c2);
 *   epi 3 / 4 (SwiGLU / GELU backward): aux = hpre; the pre-activation gradient
 *            ([rows, 2N] SwiGLU, [rows, N] GELU) is cast instead of stored (c = NULL).
 * The cast takes poff, history, hist_len, q_fmt, margin, amax_bits, scale_inv,
 * q and qt with the meaning of rhp_fp8_cast (cols = the cast output's columns,
 * the same offsets).  Results are bit for bit those of rhp_fp8_gemm followed by
 * rhp_fp8_cast of its bf16 output.  Formats: y e4m3 and q e4m3 forward, y e5m2
 * and q e5m2 backward; x e4m3.
 */
int rhp_fp8_gemm_cast(int epi, int G, const int32_t* offsets, const int32_t* poff, int64_t rows_cap, int y_fmt,
                      int x_fmt, int N, int K, int f, const void* const* y, int64_t ldy, const void* const* x,
                      int64_t ldx, int x_kn, void* const* c, int64_t ldc, const void* const* aux, int64_t ldaux,
                      const float* y_scale_inv, const float* x_scale_inv, int x_scale_stride, const float* history,
                      int hist_len, int q_fmt, int margin, uint32_t* amax_bits, float* scale_inv, void* q, void* qt,
                      hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* RESIHP_MOE_H */
