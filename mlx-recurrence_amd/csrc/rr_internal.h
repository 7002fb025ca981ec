// rr_internal.h — interfaces between the C-ABI entry points and the chunked
// (MFMA) SSD kernels.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rr {


struct Ssd2Args {
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
  float* dA;               // [H,N]
  float* dh0;              // [B,H,Dh,N] or null
  float* ws;               // backward: dA partials [B,H,nR,N]
  float* tot;              // pipelined: per-chunk delta totals [B,H,nC]
  float* agg;              // pipelined backward: chunk aggregates, then adjoints [B,H,nC,Dh,N]
  int L, H, DH, NS, nC, R;
};

// True when the chunked kernels cover this call: bf16 inputs, a head-uniform A
// (A_stride_n == 0), checkpoint interval 32, Dh in {32, 64, 128} and
// N in {16, 32, 64, 128}.
bool ssd2_supported(int dtype, int64_t L, int64_t seg, int64_t Dh, int64_t N, int64_t A_stride_n);
// Chunks per workgroup: 1 (pipelined: aggregate, pass and main kernels) or
// nC (one workgroup walks a whole head).
int ssd2_pick_run(int64_t B, int64_t H, int64_t nC, int64_t N);
int ssd2_fwd(const Ssd2Args& p, int64_t B, hipStream_t s);
// The chunked backward covers Dh in {32, 64} and N in {16, 32} (on top of
// ssd2_supported).
bool ssd2_bwd_supported(int64_t Dh, int64_t N);
// Workspace of the chunked passes: chunk aggregates + delta totals when runs
// are shorter than a head (pass 0 and 1), plus dA partials (pass 1).
size_t ssd2_ws_bytes(int64_t B, int64_t H, int64_t nC, int R, int64_t Dh, int64_t N, int pass);
void ssd2_carve_ws(Ssd2Args& a, void* ws, int64_t B, int pass);
int ssd2_bwd(const Ssd2Args& p, int64_t B, hipStream_t s);

}  // namespace rr
