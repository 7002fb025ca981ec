/*
 * recurrence.h — C ABI of librecurrence_gfx950.so, the MI355X (gfx950) kernels
 * behind the fused linear-recurrence scans ssd_scan / gla_scan / rglru_scan /
 * rotlru_scan.
 *
 * Each entry point replaces one MLX `mx.fast.metal_kernel` launcher of the
 * reference (D-CSIL/mlx-recurrence v0.3.0); the citation above each declaration
 * names it.  In the reference those launchers are Python functions that build a
 * Metal source string, JIT it and call it on MLX arrays; here they are plain C
 * functions over device pointers, so any host language with an FFI (ctypes,
 * cgo, JNI, N-API) can bind them.
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers (HBM) except where noted; every tensor is
 *     dense row-major (C-contiguous) in the layout given in its comment.
 *   - `dtype` is the element type of the large inputs (and of the gradients
 *     written for them): RR_F32, RR_BF16 or RR_F16.  Outputs y, checkpoints,
 *     initial/final states and dA_neg are always fp32; state and accumulation
 *     are fp32 (reference ssd.py:29-31, gla.py:23-26).
 *   - `seg` is validated exactly like the reference (seg > 0, L % seg == 0,
 *     lane_dim % 32 == 0; _chassis.py:92-115).  Checkpoints are written every
 *     T = rr_chunk_len(L, seg) steps: the largest power of two <= 32 dividing
 *     seg (so T divides L).  For the default seg=32, T = 32 = seg.
 *   - The caller allocates every buffer (outputs, checkpoints, workspace); the
 *     library never allocates, frees or keeps device memory.  All work is
 *     enqueued on `stream` (a hipStream_t; NULL = the default stream) and the
 *     call returns without synchronising.
 *   - Nullable arguments: h0 (zero initial state), dfinal (no cotangent on the
 *     final state), dh0 (initial-state gradient not wanted).
 *   - Return value: RR_OK, or an error code with a message available from
 *     rr_last_error() (thread-local).  Argument errors are detected before any
 *     work is enqueued.
 */
#ifndef RR_RECURRENCE_H
#define RR_RECURRENCE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RR_ABI_VERSION 12

enum rr_dtype { RR_F32 = 0, RR_BF16 = 1, RR_F16 = 2 };

enum rr_status {
  RR_OK = 0,
  RR_EINVAL = 1,      /* invalid argument (shape rule, null pointer, dtype)     */
  RR_EUNSUPPORTED = 2,/* valid call outside what the kernels implement         */
  RR_EHIP = 3,        /* HIP runtime error while enqueueing                   */
  RR_EWORKSPACE = 4   /* workspace smaller than the matching *_workspace_bytes */
};

/* ABI revision of this header (RR_ABI_VERSION). No reference counterpart. */
int rr_abi_version(void);

/* Message for the last non-RR_OK return on the calling thread.
 * Stands in for the reference's eager ValueError text (_chassis.py:104-115). */
const char* rr_last_error(void);

/* Checkpoint interval T used for (L, seg); 0 if seg/L are invalid.
 * The reference checkpoints every `seg` steps (ssd.py:103-110). */
int64_t rr_chunk_len(int64_t L, int64_t seg);

/* Errors that kernels report after their launch returned, on the current
 * device.  No reference counterpart (Metal kernels there have no runtime error
 * channel).  Waits for the device to finish (hipDeviceSynchronize), then
 * returns RR_OK, or RR_EHIP if a pass since the last call met an error whose
 * results it marked invalid (an RG-LRU / rotLRU tile hand-off wait that
 * expired: the values handed on are NaN); the message names it and the status
 * is cleared. */
int rr_async_status(void);

/* Tile schedule of the RG-LRU / rotLRU passes, for tests of the hand-off order.
 * No reference counterpart.  scan: 0 RG-LRU, 1 gated RG-LRU, 2 rotLRU (D = the
 * pair count Dp); pass 0 forward, 1 backward.  Returns the number n of
 * workgroup tickets, or -1 for invalid arguments.  When cap >= n, ticket t runs
 * step tile tile_k[t] of channel group tile_grp[t] (group = batch row * G +
 * channel tile), and *max_ckpt_row (nullable) receives the largest checkpoint
 * row b * nC + c that the backward pass reads (-1 if none or pass 0). */
int64_t rr_tile_schedule(int scan, int pass, int64_t B, int64_t L, int64_t D, int64_t seg, int dtype,
                         int32_t* tile_k, int32_t* tile_grp, int64_t* max_ckpt_row, int64_t cap);

/* ------------------------------------------------------------------ SSD --
 * u [B,L,H,Dh], delta [B,L,H], Bm/Cm [B,L,H,N] (dtype); A_neg fp32, element
 * (h, n) at A_neg[h * (A_stride_n ? N : 1) + n * A_stride_n]: A_stride_n = 1 for a
 * dense [H,N] array, 0 for one rate per head broadcast over N (Mamba-2's A,
 * as in the benchmarked SSD configurations; these calls run on the chunked
 * MFMA kernels).
 * y [B,L,H,Dh] fp32.  ckpt [B,H,nC,Dh,N] fp32, nC = L/T: the state after the
 * last step of each chunk (ckpt[:,:,nC-1] is the final state [B,H,Dh,N]).
 * h0 / dfinal / dh0: [B,H,Dh,N] fp32 (the Mamba-2 state layout of
 * ssd_scan_with_state, ssd.py:365-375).
 */

/* Workspace bytes needed by rr_ssd_fwd (pass=0) or rr_ssd_bwd (pass=1) for
 * these arguments (the kernels chosen depend on A_stride_n and dtype). */
size_t rr_ssd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N,
                              int64_t seg, int64_t A_stride_n, int dtype, int pass);

/* One past the largest workspace byte that the chunked (MFMA) SSD kernels of
 * this call write or read: the library walks the grids of the pass's kernels
 * with their own workgroup decode and slot arithmetic.  For tests that the
 * kernels stay inside rr_ssd_workspace_bytes.  No reference counterpart.
 * Returns -1 for invalid arguments or a call that the chunked bf16 kernels do
 * not run (the fp32-MFMA and VALU paths carve fixed regions of the size
 * rr_ssd_workspace_bytes returns). */
int64_t rr_ssd_workspace_extent(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N, int64_t seg,
                                int64_t A_stride_n, int dtype, int pass);

/* Replaces _ssd_forward_kernel (reference mlx_recurrence/ssd.py:54-135). */
int rr_ssd_fwd(const void* u, const void* delta, const void* Bm, const void* Cm,
               const float* A_neg, int64_t A_stride_n, int dtype, int64_t B, int64_t L, int64_t H,
               int64_t Dh, int64_t N, int64_t seg, const float* h0, float* y,
               float* ckpt, void* workspace, size_t workspace_bytes, void* stream);

/* Replaces _ssd_backward_kernel and the host mx.sum epilogue
 * (reference mlx_recurrence/ssd.py:142-307).  dy [B,L,H,Dh] fp32; gradients
 * du/ddelta/dB/dC in `dtype` with the shapes of their inputs; dA_neg fp32,
 * summed over the batch (ssd.py:305): with dA_stride_n = 1 the dense [H,N]
 * gradient (whatever A_stride_n is), with dA_stride_n = 0 the [H] gradient of a
 * per-head rate (the [H,N] one summed over n, in order of n). */
int rr_ssd_bwd(const float* dy, const float* dfinal, const void* u, const void* delta,
               const void* Bm, const void* Cm, const float* A_neg, int64_t A_stride_n, int dtype,
               int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N, int64_t seg,
               const float* h0, const float* ckpt, void* du, void* ddelta, void* dB,
               void* dC, float* dA_neg, int64_t dA_stride_n, float* dh0, void* workspace,
               size_t workspace_bytes, void* stream);

/* rr_ssd_bwd without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  The workspace is
 * a 16 MiB static device array of the library (one per device, held until the
 * process ends); the call allocates nothing.  A call whose
 * rr_ssd_workspace_bytes(..., pass = 1) exceeds 16 MiB returns
 * RR_EUNSUPPORTED (config 1 needs 36 KiB).  Every call on one device shares
 * that array: calls that overlap on one GPU (other streams or threads) race.
 * Arguments and results otherwise as rr_ssd_bwd. */
int rr_ssd_bwd_noalloc(const float* dy, const float* dfinal, const void* u, const void* delta,
                       const void* Bm, const void* Cm, const float* A_neg, int64_t A_stride_n, int dtype,
                       int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t N, int64_t seg,
                       const float* h0, const float* ckpt, void* du, void* ddelta, void* dB,
                       void* dC, float* dA_neg, int64_t dA_stride_n, float* dh0, void* stream);

/* ------------------------------------------------------------------ GLA --
 * q/k/v [B,L,H,Dh], gates [B,L,H] (dtype).  y [B,L,H,Dh] fp32.
 * ckpt [B,H,nC,Dh(j),Dh(i)] fp32: state S[i,j] stored with i fastest, so
 * ckpt[:,:,nC-1].transpose(-1,-2) is the final state [B,H,Dh(i),Dh(j)].
 * h0 / dfinal / dh0: [B,H,Dh(i),Dh(j)] fp32 (gla.py:321-329 layout).
 * bf16 inputs with T = 32 run on the chunked MFMA kernels.
 */

/* Workspace bytes needed by rr_gla_fwd (pass=0) or rr_gla_bwd (pass=1) for
 * these arguments (the kernels chosen depend on dtype). */
size_t rr_gla_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg,
                              int dtype, int pass);

/* Replaces _gla_forward_kernel (reference mlx_recurrence/gla.py:49-123). */
int rr_gla_fwd(const void* q, const void* k, const void* v, const void* gates, int dtype,
               int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg,
               const float* h0, float* y, float* ckpt, void* workspace,
               size_t workspace_bytes, void* stream);

/* Replaces _gla_backward_kernel and its mx.sum epilogue
 * (reference mlx_recurrence/gla.py:130-270). */
int rr_gla_bwd(const float* dy, const float* dfinal, const void* q, const void* k,
               const void* v, const void* gates, int dtype, int64_t B, int64_t L,
               int64_t H, int64_t Dh, int64_t seg, const float* h0, const float* ckpt,
               void* dq, void* dk, void* dv, void* dgates, float* dh0, void* workspace,
               size_t workspace_bytes, void* stream);

/* --------------------------------------------------------------- RG-LRU --
 * a, x [B,L,D] (dtype).  y [B,L,D] fp32.  ckpt [B,nC,D] fp32.
 * h0 / dfinal / dh0: [B,D] fp32.
 * The workspace carries the hand-off of states between the tiles of one pass
 * (each call clears what it uses); calls that share a workspace must not run
 * concurrently.
 */

/* Workspace bytes needed by rr_rglru_fwd (pass=0) or rr_rglru_bwd (pass=1). */
size_t rr_rglru_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t seg, int dtype, int pass);

/* Replaces _rglru_forward_kernel (reference mlx_recurrence/rglru.py:64-123). */
int rr_rglru_fwd(const void* a, const void* x, int dtype, int64_t B, int64_t L, int64_t D,
                 int64_t seg, const float* h0, float* y, float* ckpt, void* workspace,
                 size_t workspace_bytes, void* stream);

/* Replaces _rglru_backward_kernel (reference mlx_recurrence/rglru.py:130-203). */
int rr_rglru_bwd(const float* dy, const float* dfinal, const void* a, const void* x,
                 int dtype, int64_t B, int64_t L, int64_t D, int64_t seg, const float* h0,
                 const float* ckpt, void* da, void* dx, float* dh0, void* workspace,
                 size_t workspace_bytes, void* stream);

/* --------------------------------------------------------- RG-LRU, gated --
 * The RG-LRU gate math fused into the scan.  The reference computes it in MLX
 * host code before its scan kernel (mlx_recurrence/rglru.py:10-27); here the
 * kernels read the raw gates, so a(t) and x'(t) never travel through HBM.
 * Per channel d and step t:
 *   a_t = exp(-c * softplus(lam[d]) * sigmoid(r_t)),
 *   x'_t = sqrt(1 - a_t^2) * (i_t * x_t),   h_t = a_t h_{t-1} + x'_t,  y_t = h_t.
 * r, i, x [B,L,D] (dtype); lam [D] fp32; c > 0 (Griffin uses 8).  y, ckpt,
 * h0, dfinal, dh0 as for rr_rglru_*.  Gradients dr, di, dx [B,L,D] (dtype)
 * and dlam [D] fp32 (summed over batch and steps, in a fixed order).
 */

/* Workspace bytes needed by rr_rglru_gated_fwd (pass=0) or _bwd (pass=1). */
size_t rr_rglru_gated_workspace_bytes(int64_t B, int64_t L, int64_t D, int64_t seg, int dtype, int pass);

/* Replaces the gate math of rglru.py:13-14 (MLX host ops) followed by
 * _rglru_forward_kernel (rglru.py:64-123). */
int rr_rglru_gated_fwd(const void* r, const void* i, const void* x, const float* lam, float c,
                       int dtype, int64_t B, int64_t L, int64_t D, int64_t seg, const float* h0,
                       float* y, float* ckpt, void* workspace, size_t workspace_bytes, void* stream);

/* Replaces _rglru_backward_kernel (rglru.py:130-203) followed by MLX's
 * autodiff of the gate math of rglru.py:13-14. */
int rr_rglru_gated_bwd(const float* dy, const float* dfinal, const void* r, const void* i,
                       const void* x, const float* lam, float c, int dtype, int64_t B, int64_t L,
                       int64_t D, int64_t seg, const float* h0, const float* ckpt, void* dr,
                       void* di, void* dx, float* dlam, float* dh0, void* workspace,
                       size_t workspace_bytes, void* stream);

/* --------------------------------------------------------------- rotLRU --
 * a, cs, sn [B,L,Dp]; x [B,L,2*Dp] with (u,w) pairs interleaved (dtype).
 * y [B,L,2*Dp] fp32 (interleaved).  ckpt [B,nC,2*Dp] fp32.
 * h0 / dfinal / dh0: [B,2*Dp] fp32 (interleaved).  Workspace as for RG-LRU.
 */

/* Workspace bytes needed by rr_rotlru_fwd (pass=0) or rr_rotlru_bwd (pass=1). */
size_t rr_rotlru_workspace_bytes(int64_t B, int64_t L, int64_t Dp, int64_t seg, int dtype, int pass);

/* Replaces _rotlru_forward_kernel (reference mlx_recurrence/rotlru.py:80-146). */
int rr_rotlru_fwd(const void* a, const void* cs, const void* sn, const void* x, int dtype,
                  int64_t B, int64_t L, int64_t Dp, int64_t seg, const float* h0, float* y,
                  float* ckpt, void* workspace, size_t workspace_bytes, void* stream);

/* Replaces _rotlru_backward_kernel (reference mlx_recurrence/rotlru.py:153-266). */
int rr_rotlru_bwd(const float* dy, const float* dfinal, const void* a, const void* cs,
                  const void* sn, const void* x, int dtype, int64_t B, int64_t L,
                  int64_t Dp, int64_t seg, const float* h0, const float* ckpt, void* da,
                  void* dcs, void* dsn, void* dx, float* dh0, void* workspace,
                  size_t workspace_bytes, void* stream);

/* ------------------------------------------------------- rotLRU, theta --
 * The rotation passed as its angle: theta [B,L,Dp] (dtype) replaces cs and
 * sn, the kernels form cos / sin in registers (the reference computes them in
 * MLX host code, mlx_recurrence/rotlru.py:18-23, 306-317, and its kernel reads
 * both).  Other arguments and the workspace (rr_rotlru_workspace_bytes) as
 * for rr_rotlru_*; dtheta [B,L,Dp] (dtype) = -sin * dcs + cos * dsn. */
int rr_rotlru_theta_fwd(const void* a, const void* theta, const void* x, int dtype, int64_t B,
                        int64_t L, int64_t Dp, int64_t seg, const float* h0, float* y, float* ckpt,
                        void* workspace, size_t workspace_bytes, void* stream);
int rr_rotlru_theta_bwd(const float* dy, const float* dfinal, const void* a, const void* theta,
                        const void* x, int dtype, int64_t B, int64_t L, int64_t Dp, int64_t seg,
                        const float* h0, const float* ckpt, void* da, void* dtheta, void* dx,
                        float* dh0, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------- decode: one token --
 * The recurrent update of one token on a cached state, updated in place, one
 * launch per call.  The reference lists this as its next inference step
 * (docs/validation/BOTTLENECK_ANALYSIS.md:105-119: one fused kernel per layer
 * type on the final-state cache layouts of the *_scan_with_state functions,
 * ssd.py:365-375, gla.py:321-329, rglru.py:259-267, rotlru.py:323-331); the
 * arithmetic is one step of the reference recurrences (ssd.py:85-111,
 * gla.py:78-100, rglru.py:88-99, rotlru.py:101-122).  Token inputs are in
 * `dtype`; the state (fp32) is the scans' final-state layout, so a scan's
 * final state continues directly; y is fp32.  Not differentiable.
 */

/* SSD: u [B,H,Dh], delta [B,H], Bm / Cm [B,H,N] (dtype); A_neg as for
 * rr_ssd_fwd (A_stride_n 0: [H], 1: [H,N]); state [B,H,Dh,N]; y [B,H,Dh].
 * N <= 256. */
int rr_ssd_step(const void* u, const void* delta, const void* Bm, const void* Cm, const float* A_neg,
                int64_t A_stride_n, int dtype, int64_t B, int64_t H, int64_t Dh, int64_t N, float* state,
                float* y, void* stream);

/* GLA: q / k / v [B,H,Dh], gates [B,H] (dtype); state [B,H,Dh(i),Dh(j)];
 * y [B,H,Dh] (y[j] = sum_i q[i] S'[i,j], the post-update state).  Dh <= 256. */
int rr_gla_step(const void* q, const void* k, const void* v, const void* gates, int dtype, int64_t B,
                int64_t H, int64_t Dh, float* state, float* y, void* stream);

/* RG-LRU: a, x [B,D] (dtype; x the gated input, as for rr_rglru_fwd);
 * state [B,D]; y [B,D]. */
int rr_rglru_step(const void* a, const void* x, int dtype, int64_t B, int64_t D, float* state, float* y,
                  void* stream);

/* rotLRU: a, cs, sn [B,Dp]; x [B,2*Dp] interleaved (dtype); state [B,2*Dp]
 * interleaved (8-byte aligned); y [B,2*Dp]. */
int rr_rotlru_step(const void* a, const void* cs, const void* sn, const void* x, int dtype, int64_t B,
                   int64_t Dp, float* state, float* y, void* stream);

/* ------------------------------------------------------ Gated DeltaNet --
 * The reference's designed next plug-in (docs/DESIGN_gated_deltanet.md; not
 * code in the reference): the sequential kernels of its Phase 2 (:270-440,
 * :528-536) and, for bf16 / Dh 64 / T 32, the chunkwise form of its Phase 3
 * (:139-266), as a C entry pair instead of a Metal launcher.  Per (b, h):
 *   S_t = alpha_t (S_{t-1} - beta_t k_t (k_t^T S_{t-1})) + beta_t k_t v_t^T,
 *   y_t[j] = sum_i q_t[i] S_t[i,j]                           (:56-90)
 * q, k, v [B,L,H,Dh] and alpha, beta [B,L,H] (dtype; q and k L2-normalised,
 * alpha and beta pre-activated by the caller, :461-464; q and k 16-byte
 * aligned); h0 [B,H,Dh(i),Dh(j)] (nullable); y [B,L,H,Dh] fp32;
 * ckpt [B,H,L/T,Dh,Dh] fp32, the state after every T = rr_chunk_len(L, seg)
 * steps (the last is the final state).  Dh 32 or 64; T 8, 16 or 32 (seg a
 * multiple of 8).  With bf16 inputs, Dh 64 and T 32 and a workspace of
 * rr_gdn_fwd_workspace_bytes (16-byte aligned), the forward runs in the
 * chunkwise-parallel (WY) form of the design's :139-238 (its Phase 3); with
 * no workspace (NULL, 0), or for other shapes, in the sequential form.
 */
int rr_gdn_fwd(const void* q, const void* k, const void* v, const void* alpha, const void* beta, int dtype,
               int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, const float* h0, float* y, float* ckpt,
               void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of rr_gdn_fwd's chunkwise form (operand fragments of every
 * chunk, 33 KB per chunk); 0 where the forward runs sequentially (no
 * workspace needed) or for invalid arguments. */
size_t rr_gdn_fwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, int dtype);

/* Workspace bytes of rr_gdn_bwd (the adjoint at every checkpoint,
 * [B,H,L/T,Dh,Dh] fp32, then for bf16 / Dh 64 / T 32 the chunk fragments of
 * the chunkwise adjoint pass; 16-byte aligned); 0 for invalid arguments. */
size_t rr_gdn_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, int dtype);

/* Backward (:334-440): dy [B,L,H,Dh] fp32, dfinal [B,H,Dh,Dh] fp32 (nullable);
 * ckpt from rr_gdn_fwd on the same inputs; writes dq, dk, dv [B,L,H,Dh] and
 * dalpha, dbeta [B,L,H] in dtype, dh0 [B,H,Dh,Dh] fp32 (nullable).  Every
 * gradient is written (no accumulation into the buffers). */
int rr_gdn_bwd(const float* dy, const float* dfinal, const void* q, const void* k, const void* v,
               const void* alpha, const void* beta, int dtype, int64_t B, int64_t L, int64_t H, int64_t Dh,
               int64_t seg, const float* h0, const float* ckpt, void* dq, void* dk, void* dv, void* dalpha,
               void* dbeta, float* dh0, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RR_RECURRENCE_H */
