// rr_internal.h — interfaces between the C-ABI entry points and the chunked
// (MFMA) SSD and GLA kernels.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rr {

// Arguments of the chunked kernels, named for SSD.  GLA maps onto them as
// u = v, delta = gates, Bm = k, Cm = q (du = dv, ddelta = dgates, dB = dk,
// dC = dq); A, A_stride_h and dA are unused there.
struct ChunkArgs {
  const uint16_t* u;       // [B,L,H,Dh] bf16
  const uint16_t* delta;   // [B,L,H]
  const uint16_t* Bm;      // [B,L,H,N]
  const uint16_t* Cm;      // [B,L,H,N]
  const float* A;          // head-uniform decay rate: A[h * A_stride_h]
  int64_t A_stride_h;
  const float* h0;         // [B,H,Dh,N] or null
  float* y;                // [B,L,H,Dh]
  float* ckpt;             // [B,H,nC,Dh,N]
  // backward
  const float* dy;         // [B,L,H,Dh]
  const float* dfinal;     // [B,H,Dh,N] or null
  uint16_t* du;
  uint16_t* ddelta;
  uint16_t* dB;
  uint16_t* dC;
  float* dA;               // [H,N], or [H] (summed over n) when dA_sn == 0
  int dA_sn;               // n-stride of dA: 1 dense [H,N], 0 per head [H]
  float* dh0;              // [B,H,Dh,N] or null
  float* ws;               // SSD backward: dA partials [B,H,nR,N]
  float* tot;              // pipelined: per-chunk decay gam_31 [B,H,nC]
  float* agg;              // pipelined backward: chunk aggregates, then adjoints [B,H,nC,Dh,N]
  int B, L, H, DH, NS, nC;
  int R;                   // chunks per workgroup: nC (whole-head mode), 2 (pair mode) or 1
  int mode;                // rr::chunked::Mode (rr_chunked.h)
};

// Mode of the SSD chunked kernels for pass 0 (forward) or 1 (backward), B*H
// heads of nC chunks of a Dh x N state: a whole head per workgroup for the
// forward when the heads alone fill the GPU (and for either pass when a 1-D
// per-chunk grid would exceed 2^31 workgroups); else one workgroup per chunk,
// with the entering states formed directly (nC <= 4 with Dh * N <= 64 * 64;
// nC <= 16 with Dh 128, N 64 and at most 768 chunk workgroups), from the chunk
// aggregates (nC <= 16, N <= 32) or by the pipelined aggregate and state-pass
// kernels.
int chunked_mode(int64_t B, int64_t H, int64_t nC, int64_t Dh, int64_t N, int pass);
int chunked_run(int mode, int64_t nC);   // ChunkArgs::R of a mode

// ------------------------------------------------------------------ SSD
// True when the chunked kernels cover this call: bf16 inputs, a head-uniform A
// (A_stride_n == 0), checkpoint interval 32, Dh in {32, 64, 128} and
// N in {16, 32, 64, 128}.
bool ssd2_supported(int dtype, int64_t L, int64_t seg, int64_t Dh, int64_t N, int64_t A_stride_n);
int ssd2_fwd(const ChunkArgs& p, int64_t B, hipStream_t s);
// The chunked backward covers Dh in {32, 64}, and Dh = 128 with N in {64, 128}
// (on top of ssd2_supported).
bool ssd2_bwd_supported(int64_t Dh, int64_t N);
// Workspace of the chunked passes: chunk decays and (backward) chunk adjoints
// in the pipelined mode, plus dA partials (pass 1).
size_t ssd2_ws_bytes(int64_t B, int64_t H, int64_t nC, int mode, int64_t Dh, int64_t N, int pass);
void ssd2_carve_ws(ChunkArgs& a, void* ws, int64_t B, int pass);
// One past the largest workspace byte that the chunked SSD kernels of a pass
// write or read, walked over their grids with the kernels' own decode and slot
// arithmetic (a host-side bound for tests).
int64_t ssd2_ws_extent(int64_t B, int64_t H, int64_t nC, int mode, int64_t Dh, int64_t N, int pass);
int ssd2_bwd(const ChunkArgs& p, int64_t B, hipStream_t s);

// ------------------------------------------------------------------ GLA
// True when the chunked GLA kernels cover this call (pass 0 forward, 1
// backward): bf16 inputs, checkpoint interval 32, Dh in {32, 64, 128}, and a
// 1-D grid of one workgroup per
// chunk below 2^31 (direct or pipelined modes; whole heads run with
// B * H >= 512: the forward always, the backward up to 16 chunks).
bool gla2_supported(int dtype, int64_t B, int64_t L, int64_t H, int64_t seg, int64_t Dh, int pass);
int gla2_mode(int64_t B, int64_t H, int64_t nC, int64_t Dh, int pass);
// Workspace of the pipelined mode: chunk decays [B,H,nC] (both passes) and
// the backward chunk adjoints [B,H,nC,Dh,Dh] (pass 1); none in the direct and
// whole-head modes.
size_t gla2_ws_bytes(int64_t B, int64_t H, int64_t nC, int64_t Dh, int pass);
void gla2_carve_ws(ChunkArgs& a, void* ws, int64_t B, int pass);
int gla2_fwd(const ChunkArgs& p, int64_t B, hipStream_t s);
int gla2_bwd(const ChunkArgs& p, int64_t B, hipStream_t s);

// Forward with every chunk of a head resident in one workgroup per 16-column
// slice of the state's d axis (resident.hip): nC <= 16, Dh % 16 == 0,
// N in {16, 32, 64} (GLA: N = Dh in {32, 64}), 16 nC >= N.
bool res_fwd_supported(int64_t B, int64_t H, int64_t nC, int64_t Dh, int64_t N);
int res_fwd(const ChunkArgs& p, int64_t B, hipStream_t s, bool gla);

// Gated DeltaNet forward in chunkwise (WY) form (gdn_chunk.hip): bf16, Dh 64,
// checkpoint interval 32; the workspace holds every chunk's operand fragments.
bool gdn_chunk_supported(int dtype, int64_t Dh, int64_t T);
size_t gdn_chunk_ws_bytes(int64_t B, int64_t L, int64_t H);
int gdn_chunk_fwd(const void* q, const void* k, const void* v, const void* alpha, const void* beta, int64_t B,
                  int64_t L, int64_t H, const float* h0, float* y, float* ckpt, void* workspace, hipStream_t s);
// The backward's adjoint pass in the same form: the adjoint at every chunk
// end (adjck [B,H,nC,Dh,Dh], as the sequential pass writes it) and dh0.
size_t gdn_chunk_bwd_ws_bytes(int64_t B, int64_t L, int64_t H);
int gdn_chunk_adjoint(const void* q, const void* k, const void* v, const void* alpha, const void* beta, const float* dy,
                      const float* dfinal, int64_t B, int64_t L, int64_t H, float* adjck, float* dh0, void* packs,
                      hipStream_t s);
// The gradient pass in chunkwise form, every chunk at once, from the forward
// and adjoint checkpoints.
int gdn_chunk_grad(const float* dy, const void* q, const void* k, const void* v, const void* alpha, const void* beta,
                   const float* h0, const float* ckpt, const float* adjck, void* dq, void* dk, void* dv, void* dalpha,
                   void* dbeta, int64_t B, int64_t L, int64_t H, hipStream_t s);

// ------------------------------------------------------------------ SSD, rate per (head, n)
// Chunked SSD for A_neg [H, N] (any input dtype) and for fp32 / fp16 inputs
// with a per-head rate (ssd_dense.hip): one workgroup per 32-step chunk,
// contractions on the fp32 MFMA.  It writes every chunk's map (mapE
// [B,H,nC,Dh,N], mapP [B,H,nC,N]), and ssd_dense_compose walks them into ckpt
// (forward) and lamws (backward).
struct DenseArgs {
  const void* u;           // [B,L,H,Dh] of the input dtype
  const void* delta;       // [B,L,H]
  const void* Bm;          // [B,L,H,N]
  const void* Cm;          // [B,L,H,N]
  const float* A;          // A[h * a_sh + n * a_sn]
  int64_t a_sh, a_sn;
  const float* h0;         // [B,H,Dh,N] or null
  const float* ckpt;       // [B,H,nC,Dh,N]: the state after each chunk
  const float* lamws;      // [B,H,nC,Dh,N]: the adjoint flowing into each chunk's end
  const float* dy;         // [B,L,H,Dh]
  float* y;                // [B,L,H,Dh]
  void* du;                // gradients, of the input dtype
  void* ddelta;
  void* dB;
  void* dC;
  float* gA_part;          // [H][B * nC][N]: dA of each chunk
  float* mapE;
  float* mapP;
  int B, L, H, DH, NS, nC;
};
enum DenseKernel { kDenseMapsFwd = 0, kDenseMapsBwd = 1, kDenseOut = 2, kDenseGrad = 3 };
// True when the chunk kernels cover the call: checkpoint interval T = 32,
// Dh in {32, 64} with N in {16, 32}, Dh 64 with N 64, or Dh 128 with N in
// {16, 32, 64} (the wide ones streamed in blocks of d), and a 1-D grid of one
// workgroup per chunk.
bool ssd_dense_supported(int64_t T, int64_t Dh, int64_t N, int64_t B, int64_t H, int64_t nC);
int ssd_dense_launch(const DenseArgs& a, int dtype, int what, hipStream_t s);
// GLA for fp32 / fp16 inputs (and bf16 where the chunked kernels do not run),
// T = 32, Dh in {32, 64, 128} (gla_dense.hip): the same three-kernel scheme, the
// maps in the layout dense_compose walks (mapP: gam_31 in every column).
struct GlaDenseArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const float* h0;      // [B,H,Dh,Dh] as [i][j], or null
  const float* ckpt;    // [B,H,nC,Dh,Dh] as [j][i]
  const float* lamws;   // [B,H,nC,Dh,Dh] as [j][i]
  const float* dy;      // [B,L,H,Dh]
  float* y;
  void* dq;
  void* dk;
  void* dv;
  void* dg;
  float* mapE;
  float* mapP;
  int B, L, H, D, nC;
};
bool gla_dense_supported(int64_t T, int64_t Dh, int64_t B, int64_t H, int64_t nC);
int gla_dense_launch(const GlaDenseArgs& a, int dtype, int what, hipStream_t s);

// The walk over the chunk maps (SSD and GLA): forward x0 = h0, out = ckpt (the
// state after each chunk); backward x0 = dfinal, out = lamws (the adjoint
// flowing into each chunk's end), xlast = dh0.  x0 and xlast may be null; they
// are [n][d] for GLA (the reference's [i, j]), [d][n] for SSD.
int dense_compose(const float* mapE, const float* mapP, const float* x0, float* out, float* xlast, int64_t B,
                  int64_t H, int64_t Dh, int64_t N, int64_t nC, bool bwd, bool gla, hipStream_t s);

// Backward of the chunked kernels with column-owned state blocks (GLA: Dh in
// {32, 64, 128}; SSD: Dh in {32, 64, 128}, N in {64, 128}; chunked_bwd.hip).  SSD
// leaves per-run dA partials in p.ws for the caller's reduction.
int chunked_bwd_cols(const ChunkArgs& p, int64_t B, hipStream_t s, bool gla);

}  // namespace rr
