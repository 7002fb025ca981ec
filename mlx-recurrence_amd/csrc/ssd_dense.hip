// ssd_dense.hip — SSD with a decay rate per (head, state column n) — the
// reference's own A_neg [H, N] — in chunked form, contractions on the fp32
// MFMA, for chunks of 32 steps.  Also taken by fp32 / fp16
// inputs with a per-head rate (the chunked kernels of rr_chunked.h take bf16
// only).
//
// Per chunk of one (batch, head), steps t, s < 32, cd = in-chunk cumulative
// delta, E[t,n] = exp(A_n cd_t), m31[s,n] = exp(A_n (cd_31 - cd_s)) and
// M_n[t,s] = exp(A_n (cd_t - cd_s)) for t >= s (0 else) — the matrix form of
// the reference's per-step recurrence and adjoint (ssd.py:85-111, 203-268):
//   chunk map, forward:  S  = U^T diag(delta) (m31 o B); the state after the
//                        chunk is E_31 o h_in + S
//   chunk map, backward: S' = dY^T (E o C); the adjoint handed to the chunk
//                        before is E_31 o lam + S'
//   Y   = (W o delta_s) U + (C o E) h_in^T,   W[t,s] = sum_n C_t[n] B_s[n] M_n[t,s]
//   du  = diag(delta) (W^T dY + (B o m31) lam^T)
//   with G2 = dY U^T, GH = dY h_in, UL = U lam, F_n[t,s] = M_n[t,s] G2[t,s]:
//   ZF[s,n]  = sum_t F_n[t,s] C_t[n];          Z = ZF + m31 o UL;  dB = diag(delta) Z
//   dC2[t,n] = sum_s F_n[t,s] delta_s B_s[n];  dC = E o GH + dC2
//   D[t,n]   = sum_{t'>=t} (E C GH)[t',n] + R[t,n] + E_31[n] tr[n] + sum_{s<t} (m31 delta B UL)[s,n],
//     R[t,n] = sum_{tau>=t} (C dC2 - delta B ZF)[tau,n]  (the dominance sum
//              sum_{t'>=t>s} F_n[t',s] delta_s B_s[n] C_t'[n], telescoped), tr = sum_d lam o h_in
//   d(delta)_t = sum_n (A_n D[t,n] + B_t[n] Z[t,n])
//   dA[n]    = sum_t delta_t D[t,n], summed here with each term's weight formed
//              exactly:  sum_t (E C GH)[t,n] cd_t + cd_31 E_31[n] tr[n]
//              + sum_s (m31 delta B UL)[s,n] (cd_31 - cd_s) + sum_s delta_s B_s[n] ZW[s,n],
//     ZW[s,n] = sum_t F_n[t,s] C_t[n] (cd_t - cd_s).  (The suffix sum R cancels
//     to R[0] = 0 from O(1) terms; summed over t for dA that cancellation would
//     cost ~1e-5 of dA's scale in fp32, the weighted form none.)
// where h_in is the state entering the chunk and lam the adjoint flowing into
// its end from the later chunks, both from dense_compose_kernel's walk over
// the chunk maps.  D[t,n] is dec_t[n] sum_d lam_t h_{t-1}, the
// quantity both d(delta) and dA need, formed without dividing by a decay.
// (Derived from the per-step adjoint and checked in float64 against the oracle
// before this code; the GPU parity tests check it against the oracle.)
//
// Work split: one workgroup per chunk, three kernels per pass (chunk maps;
// the walk over them, one thread per state element; every chunk's outputs or
// gradients: four waves for the maps and outputs, eight for the gradients,
// sixteen for the gradients of wide states).  Each workgroup issues all of its
// global loads before it writes any of them to LDS (one memory latency per
// chunk, not one per staged row).  The inputs and the intermediates live in
// LDS as fp32, and the contractions run on the fp32 MFMA (fp32 products and
// sums: fp32 inputs keep fp32 accuracy, where a bf16 hi + lo operand split
// would leave ~2^-18 per product).  The per-n masked sums W, ZF, ZW and dC2 are
// masked MFMA products of the factored decays where the chunk's factors stay
// in range, and VALU sums with an exponential per (t, s, n) in steep chunks
// (see Factor below).  Wide states (Dh 128, N 64) stream d in blocks (see the
// wide-state kernels at the end).
#include "rr_common.h"
#include "rr_dense.h"
#include "rr_internal.h"
#include "rr_mfma.h"

namespace {

using namespace rr::dense;

template <typename InT>
struct DenseArgsT {
  const InT* u;
  const InT* delta;
  const InT* Bm;
  const InT* Cm;
  const float* A;
  int64_t a_sh, a_sn;      // A[h * a_sh + n * a_sn]
  const float* h0;         // [B,H,Dh,N] or null
  const float* ckpt;       // [B,H,nC,Dh,N]: the state after each chunk
  const float* lamws;      // [B,H,nC,Dh,N]: the adjoint flowing into each chunk's end
  const float* dy;         // [B,L,H,Dh]
  float* y;
  InT* du;
  InT* ddelta;
  InT* dB;
  InT* dC;
  float* gA_part;          // [H][B * nC][N]: dA of each chunk
  float* mapE;             // [B,H,nC,Dh,N]
  float* mapP;             // [B,H,nC,N]
  int B, L, H, DH, NS, nC;
};

template <typename InT>
__device__ __forceinline__ ChunkPos chunk_pos(const DenseArgsT<InT>& p) {
  return rr::dense::chunk_pos(p.H, p.L, p.nC);
}

// The decays of a chunk factor as M_n[t,s] = Ef[t,n] / Ef[s,n] with
// Ef[t,n] = exp(a_n (cd_t - cm)), cm the middle of the range of cd (and 0).
// Where every Ef and 1 / Ef lies within e^{+-80} (far inside fp32's normal
// range), the masked sums over s, t of the backward and W are MFMA products of
// ECt = Ef o C and BEi = B / Ef; else ("steep" chunks) they are formed with an
// exponential per (t, s, n).  kFactorLimit bounds max_n |a_n| * half-range.
constexpr float kFactorLimit = 80.f;
struct Factor {
  float cm;
  float fast;   // 1: the factored form holds
};

// Step scalars of the chunk: delta (thread t < 32) and the rates (thread
// n < NS) are loaded by the caller with the other inputs; this writes them to
// LDS, forms cd (wave 0's prefix sum) and the factor scale, then E[t,n],
// m31[t,n] and (in factored chunks) ECt, BEi, as requested (null: not wanted).
// Cm and Bm must be in LDS before the call when ECt / BEi are wanted.
template <int NS, int PN, int NT = 256>
__device__ __forceinline__ void step_scalars(float dv, float av, float* del, float* cd, float* a, Factor* fac,
                                             float (*E)[PN], float (*m31)[PN], float (*ECt)[PN], float (*BEi)[PN],
                                             const float (*Cm)[PN], const float (*Bm)[PN], int tid) {
  if (tid < Q) del[tid] = dv;
  if (tid < NS) a[tid] = av;
  if (tid < 64) {   // wave 0; lanes >= 32 take cd = 0 (the chunk's start)
    const float c = rr::prefix32_sum(tid < Q ? dv : 0.f);
    if (tid < Q) cd[tid] = c;
    if (fac != nullptr) {
      const float cmax = wave_max(c), cmin = -wave_max(-c), amax = wave_max(fabsf(av));
      if (tid == 0) {
        fac->cm = 0.5f * (cmax + cmin);
        fac->fast = amax * (0.5f * (cmax - cmin)) <= kFactorLimit ? 1.f : 0.f;
      }
    }
  }
  __syncthreads();
  const float c31 = cd[Q - 1];
  const bool fast = fac != nullptr && __builtin_amdgcn_readfirstlane(__float_as_int(fac->fast)) != 0;
  const float cm = fac != nullptr ? fac->cm : 0.f;
#pragma unroll
  for (int j = 0; j < (Q * NS + NT - 1) / NT; ++j) {
    const int i = tid + NT * j, t = i / NS, n = i % NS;
    if (Q * NS % NT != 0 && i >= Q * NS) break;
    const float an = a[n], ct = cd[t];
    if (E != nullptr) E[t][n] = __expf(an * ct);
    if (m31 != nullptr) m31[t][n] = __expf(an * (c31 - ct));
    if (ECt != nullptr && fast) {
      ECt[t][n] = __expf(an * (ct - cm)) * Cm[t][n];
      BEi[t][n] = __expf(-an * (ct - cm)) * Bm[t][n];
    }
  }
}

// The chunk's delta (thread t < 32) and rate (thread n < NS), loaded with the
// slabs.
template <int NS, typename InT>
__device__ __forceinline__ void load_step(const DenseArgsT<InT>& p, const ChunkPos& cp, int tid, float& dv, float& av) {
  dv = rr::ld(p.delta, (cp.row0 + (tid & (Q - 1))) * p.H + cp.h);
  av = p.A[(int64_t)cp.h * p.a_sh + (int64_t)(tid & (NS - 1)) * p.a_sn];
}

// W[t,s] = sum_n C_t[n] B_s[n] M_n[t,s] (t >= s; 0 else) with an exponential
// per (t, s, n): one thread per (t, s).
template <int NS, int PN, int PQ, int NT = 256>
__device__ __forceinline__ void form_w(float (*W)[PQ], const float (*Cm)[PN], const float (*Bm)[PN], const float* cd,
                                       const float* a, int tid) {
#pragma unroll
  for (int j = 0; j < (Q * Q + NT - 1) / NT; ++j) {
    const int i = tid + NT * j, t = i / Q, s = i % Q;
    if (Q * Q % NT != 0 && i >= Q * Q) break;
    const bool keep = t >= s;
    const float dc = cd[t] - cd[s];
    float w = 0.f;
#pragma unroll
    for (int n = 0; n < NS; ++n) w += Cm[t][n] * Bm[s][n] * kept_exp(keep, a[n] * dc);
    W[t][s] = w;
  }
}

// W of a factored chunk: W[t,s] = sum_n ECt[t,n] BEi[s,n] (t >= s; 0 else) on
// MFMA, 16 x 16 block (t0, s0) by one wave.
template <int NS, int PN, int PQ>
__device__ __forceinline__ void form_w_block(float (*W)[PQ], const float (*ECt)[PN], const float (*BEi)[PN], int t0,
                                             int s0, int lane) {
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (t0 >= s0)
    acc = mm16<NS>([&](int r, int k) { return ECt[t0 + r][k]; }, [&](int k, int c) { return BEi[s0 + c][k]; }, lane,
                   acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = t0 + 4 * (lane >> 4) + r, s = s0 + (lane & 15);
    W[t][s] = t >= s ? acc[r] : 0.f;
  }
}

// ------------------------------------------------------------------ chunk maps
// Forward: S[d][n] = sum_s u_s[d] delta_s m31[s,n] B_s[n]; backward:
// S'[d][n] = sum_t dY_t[d] E[t,n] C_t[n]; P[n] = E[31, n].  (The layout
// dense_compose_kernel walks.)
template <int DH, int NS>
struct alignas(16) MapSmem {
  static constexpr int PD = DH + 4, PN = NS + 4;
  float X[Q][PD];    // u (forward) or dY (backward) [t][d]
  float V[Q][PN];    // B (forward) or C (backward)
  float F[Q][PN];    // m31 (forward) or E (backward)
  float del[Q], cd[Q], a[NS];
};

template <typename InT, int DH, int NS, bool BWD>
__global__ __launch_bounds__(256) void dense_map_kernel(DenseArgsT<InT> p) {
  using S = MapSmem<DH, NS>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkPos cp = chunk_pos(p);
  const int64_t xoff = (cp.row0 * p.H + cp.h) * DH, voff = (cp.row0 * p.H + cp.h) * NS;
  Slab<Q, DH> X;
  Slab<Q, NS> V;
  float dv, av;
  if constexpr (BWD) {
    X.load(p.dy + xoff, (int64_t)p.H * DH, tid);
    V.load(p.Cm + voff, (int64_t)p.H * NS, tid);
  } else {
    X.load(p.u + xoff, (int64_t)p.H * DH, tid);
    V.load(p.Bm + voff, (int64_t)p.H * NS, tid);
  }
  load_step<NS>(p, cp, tid, dv, av);
  X.store(sm.X, tid);
  V.store(sm.V, tid);
  if constexpr (BWD)
    step_scalars<NS, S::PN>(dv, av, sm.del, sm.cd, sm.a, nullptr, sm.F, nullptr, nullptr, nullptr, nullptr, nullptr, tid);
  else
    step_scalars<NS, S::PN>(dv, av, sm.del, sm.cd, sm.a, nullptr, nullptr, sm.F, nullptr, nullptr, nullptr, nullptr, tid);
  __syncthreads();
  constexpr int NBD = DH / 16, NBN = NS / 16;
  float* dst = p.mapE + ((cp.bh * p.nC + cp.c) * DH) * NS;
  for (int blk = w; blk < NBD * NBN; blk += 4) {
    const int d0 = 16 * (blk / NBN), n0 = 16 * (blk % NBN);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (BWD) {
      acc = mm16<Q>([&](int r, int k) { return sm.X[k][d0 + r]; },
                    [&](int k, int c) { return sm.F[k][n0 + c] * sm.V[k][n0 + c]; }, lane, acc);
    } else {
      acc = mm16<Q>([&](int r, int k) { return sm.X[k][d0 + r]; },
                    [&](int k, int c) { return sm.del[k] * sm.F[k][n0 + c] * sm.V[k][n0 + c]; }, lane, acc);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(d0 + 4 * (lane >> 4) + r) * NS + n0 + (lane & 15)] = acc[r];
  }
  if (tid < NS) p.mapP[(cp.bh * p.nC + cp.c) * NS + tid] = __expf(sm.a[tid] * sm.cd[Q - 1]);
}

// ------------------------------------------------------------------ forward y
template <int DH, int NS>
struct alignas(16) OutSmem {
  static constexpr int PD = DH + 4, PN = NS + 4, PQ = Q + 4;
  float U[Q][PD];
  float Bm[Q][PN], Cm[Q][PN], E[Q][PN];
  float hin[DH][PN];
  float W[Q][PQ];
  float ECt[Q][PN], BEi[Q][PN];
  float del[Q], cd[Q], a[NS];
  Factor fac;
};

constexpr int kOutThreads = 512, kOutWaves = kOutThreads / 64;   // eight waves: the Y blocks spread out
template <typename InT, int DH, int NS>
__global__ __launch_bounds__(kOutThreads) void dense_out_kernel(DenseArgsT<InT> p) {
  constexpr int NT = kOutThreads, NW = kOutWaves;
  using S = OutSmem<DH, NS>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkPos cp = chunk_pos(p);
  const int64_t xoff = (cp.row0 * p.H + cp.h) * DH, voff = (cp.row0 * p.H + cp.h) * NS;
  Slab<Q, DH, NT> U;
  Slab<Q, NS, NT> Bv, Cv;
  Slab<DH, NS, NT> Hs;   // the state entering the chunk: checkpoint c - 1, h0 or zero
  float dv, av;
  U.load(p.u + xoff, (int64_t)p.H * DH, tid);
  Bv.load(p.Bm + voff, (int64_t)p.H * NS, tid);
  Cv.load(p.Cm + voff, (int64_t)p.H * NS, tid);
  if (cp.c > 0) Hs.load(p.ckpt + (cp.bh * p.nC + cp.c - 1) * DH * NS, NS, tid);
  else if (p.h0 != nullptr) Hs.load(p.h0 + cp.bh * DH * NS, NS, tid);
  else Hs.zero();
  load_step<NS>(p, cp, tid, dv, av);
  U.store(sm.U, tid);
  Bv.store(sm.Bm, tid);
  Cv.store(sm.Cm, tid);
  Hs.store(sm.hin, tid);
  step_scalars<NS, S::PN, NT>(dv, av, sm.del, sm.cd, sm.a, &sm.fac, sm.E, nullptr, sm.ECt, sm.BEi, sm.Cm, sm.Bm, tid);
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane(__float_as_int(sm.fac.fast)) != 0) {
    if (w < 4) form_w_block<NS, S::PN, S::PQ>(sm.W, sm.ECt, sm.BEi, 16 * (w >> 1), 16 * (w & 1), lane);
  } else {
    form_w<NS, S::PN, S::PQ, NT>(sm.W, sm.Cm, sm.Bm, sm.cd, sm.a, tid);
  }
  __syncthreads();
  // Y [t][d] = sum_s W[t][s] delta_s U[s][d] + sum_n C[t][n] E[t][n] hin[d][n]
  constexpr int NBD = DH / 16;
  for (int blk = w; blk < 2 * NBD; blk += NW) {
    const int t0 = 16 * (blk / NBD), d0 = 16 * (blk % NBD);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16<Q>([&](int r, int k) { return sm.W[t0 + r][k] * sm.del[k]; },
                  [&](int k, int c) { return sm.U[k][d0 + c]; }, lane, acc);
    acc = mm16<NS>([&](int r, int k) { return sm.Cm[t0 + r][k] * sm.E[t0 + r][k]; },
                   [&](int k, int c) { return sm.hin[d0 + c][k]; }, lane, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * (lane >> 4) + r;
      p.y[((cp.row0 + t) * p.H + cp.h) * DH + d0 + (lane & 15)] = acc[r];
    }
  }
}

// The masked sums of the backward: ZF[s,n] = sum_{t>=s} F_n[t,s] C_t[n], ZW (the
// same weighted by cd_t - cd_s), dC2[t,n] = sum_{s<=t} F_n[t,s] delta_s B_s[n],
// and (WITH_W) W of a factored chunk, from G2, the step scalars and (factored)
// ECt / BEi or (steep) B, C.  S: a gradient kernel's LDS (same member names).
template <int NS, int NT, int NW, bool WITH_W, class S>
__device__ __forceinline__ void masked_sums(S& sm, bool fast, int tid, int w, int lane) {
  constexpr int NBN = NS / 16, W0 = WITH_W ? 4 : 0;
  if (fast) {
    // Ef_s^-1 G2m^T ECt, the same with G2m o (cd_t - cd_s), Ef_t G2m (delta BEi):
    // masked MFMA products (G2m: G2 for t >= s, 0 else; the k-range of a block
    // skips its all-zero part).  Blocks: W's four, then ZF, ZW, dC2 (2 NBN each).
    const float cm = sm.fac.cm;
    for (int blk = w; blk < W0 + 6 * NBN; blk += NW) {
      if (blk < W0) {
        form_w_block<NS, S::PN, S::PQ>(sm.W, sm.ECt, sm.BEi, 16 * (blk >> 1), 16 * (blk & 1), lane);
        continue;
      }
      const int kind = (blk - W0) / (2 * NBN), rem = (blk - W0) % (2 * NBN);
      const int r0 = 16 * (rem / NBN), n0 = 16 * (rem % NBN);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      const auto ect = [&](int k, int c) { return sm.ECt[k][n0 + c]; };
      if (kind == 0) {          // ZF, rows s
        const auto fa = [&](int r, int k) { return k >= r0 + r ? sm.G2[k][r0 + r] : 0.f; };
        acc = r0 == 0 ? mm16r<0, Q>(fa, ect, lane, acc) : mm16r<16, Q>(fa, ect, lane, acc);
      } else if (kind == 1) {   // ZW, rows s
        const auto fa = [&](int r, int k) {
          const int s = r0 + r;
          return k >= s ? sm.G2[k][s] * (sm.cd[k] - sm.cd[s]) : 0.f;
        };
        acc = r0 == 0 ? mm16r<0, Q>(fa, ect, lane, acc) : mm16r<16, Q>(fa, ect, lane, acc);
      } else {                  // dC2, rows t
        const auto fa = [&](int r, int k) { return k <= r0 + r ? sm.G2[r0 + r][k] : 0.f; };
        const auto fb = [&](int k, int c) { return sm.del[k] * sm.BEi[k][n0 + c]; };
        acc = r0 == 0 ? mm16r<0, 16>(fa, fb, lane, acc) : mm16r<0, Q>(fa, fb, lane, acc);
      }
      const int n = n0 + (lane & 15);
      const float an = sm.a[n];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = r0 + 4 * (lane >> 4) + r;
        const float x = an * (sm.cd[row] - cm);
        if (kind == 0) sm.ZF[row][n] = acc[r] * __expf(-x);
        else if (kind == 1) sm.ZW[row][n] = acc[r] * __expf(-x);
        else sm.dC2[row][n] = acc[r] * __expf(x);
      }
    }
  } else {
#pragma unroll
    for (int jj = 0; jj < (Q * NS + NT - 1) / NT; ++jj) {
      const int i = tid + NT * jj, j = i / NS, n = i % NS;
      if (Q * NS % NT != 0 && i >= Q * NS) break;
      const float an = sm.a[n], cj = sm.cd[j];
      float zf = 0.f, zw = 0.f, dc2 = 0.f;
#pragma unroll 8
      for (int k = 0; k < Q; ++k) {
        // ZF, ZW: s = j, t = k; dC2: t = j, s = k
        const float dk = sm.cd[k] - cj;
        const float g = sm.G2[k][j] * kept_exp(k >= j, an * dk) * sm.Cm[k][n];
        zf += g;
        zw += g * dk;
        dc2 += sm.G2[j][k] * kept_exp(k <= j, -an * dk) * sm.del[k] * sm.Bm[k][n];
      }
      sm.ZF[j][n] = zf;
      sm.ZW[j][n] = zw;
      sm.dC2[j][n] = dc2;
    }
  }
}

// The backward's epilogue: dB = delta Z, dC = E GH + dC2, then D[t,n] by
// scans over t, this chunk's dA and d(delta) (needs ZF, ZW, dC2, GH, UL, tr).
template <int NS, int NT, int NW, class S, typename InT>
__device__ __forceinline__ void grad_epilogue(const DenseArgsT<InT>& p, S& sm, const ChunkPos& cp, int tid, int w,
                                              int lane) {
  // dB = delta Z, dC = E GH + dC2
#pragma unroll
  for (int jj = 0; jj < (Q * NS + NT - 1) / NT; ++jj) {
    const int i = tid + NT * jj, t = i / NS, n = i % NS;
    if (Q * NS % NT != 0 && i >= Q * NS) break;
    const int64_t gi = ((cp.row0 + t) * p.H + cp.h) * NS + n;
    rr::st(p.dB, gi, sm.del[t] * (sm.ZF[t][n] + sm.m31[t][n] * sm.UL[t][n]));
    rr::st(p.dC, gi, sm.E[t][n] * sm.GH[t][n] + sm.dC2[t][n]);
  }
  // D[t,n] by scans over t (lanes t of a half-wave, one n per half-wave); dA
  // of this chunk and the per-(wave, half) partials of d(delta)
  {
    const int t = lane & (Q - 1), hf = lane >> 5;
    float ddp = 0.f;
    for (int n2 = 2 * w; n2 < NS; n2 += 2 * NW) {
      const int n = n2 + hf;   // NS even: n < NS
      const float e = sm.E[t][n], c = sm.Cm[t][n], bd = sm.del[t] * sm.Bm[t][n], zf = sm.ZF[t][n];
      const float x = e * c * sm.GH[t][n];
      const float rt = c * sm.dC2[t][n] - bd * zf;
      const float yv = sm.m31[t][n] * bd * sm.UL[t][n];
      const float px = rr::prefix32_sum(x), pr = rr::prefix32_sum(rt), py = rr::prefix32_sum(yv);
      const float tx = __shfl(px, 31 + 32 * hf), trr = __shfl(pr, 31 + 32 * hf);
      const float D = (tx - px + x) + (trr - pr + rt) + sm.E[Q - 1][n] * sm.tr[n] + (py - yv);
      const float ct = sm.cd[t], c31 = sm.cd[Q - 1];
      const float da = rr::prefix32_sum(x * ct + yv * (c31 - ct) + bd * sm.ZW[t][n]);
      if (t == Q - 1)
        p.gA_part[((int64_t)cp.h * (p.B * p.nC) + (int64_t)cp.b * p.nC + cp.c) * NS + n] =
            da + c31 * sm.E[Q - 1][n] * sm.tr[n];
      ddp += sm.a[n] * D + sm.Bm[t][n] * (zf + sm.m31[t][n] * sm.UL[t][n]);
    }
    sm.ddp[w][hf][t] = ddp;
  }
  __syncthreads();
  if (tid < Q) {
    float s = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) s += sm.ddp[ww][0][tid] + sm.ddp[ww][1][tid];
    rr::st(p.ddelta, (cp.row0 + tid) * p.H + cp.h, s);
  }
}


// ------------------------------------------------------------------ backward
// Eight waves per chunk: the LDS of a chunk allows two workgroups per CU, and
// the phases below are LDS-latency bound, so more waves per workgroup keep the
// SIMDs busy.
constexpr int kGradThreads = 512, kGradWaves = kGradThreads / 64;
template <int DH, int NS>
struct alignas(16) GradSmem {
  static constexpr int PD = DH + 4, PN = NS + 4, PQ = Q + 4;
  float U[Q][PD];       // u [s][d]
  float G[Q][PD];       // dY [t][d]
  float Bm[Q][PN], Cm[Q][PN];
  float E[Q][PN], m31[Q][PN];
  float hin[DH][PN], lam[DH][PN];
  float G2[Q][PQ];      // dY U^T [t][s]
  float W[Q][PQ];       // W [t][s]
  float GH[Q][PN], UL[Q][PN], ZF[Q][PN], ZW[Q][PN], dC2[Q][PN];
  float ECt[Q][PN], BEi[Q][PN];
  float del[Q], cd[Q], a[NS], trp[kGradThreads / NS][NS], tr[NS];
  float ddp[kGradWaves][2][Q];   // per-(wave, half) partials of d(delta)
  Factor fac;
};

template <typename InT, int DH, int NS>
__global__ __launch_bounds__(kGradThreads) void dense_grad_kernel(DenseArgsT<InT> p) {
  constexpr int NT = kGradThreads, NW = kGradWaves;
  using S = GradSmem<DH, NS>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkPos cp = chunk_pos(p);
  // ---- A: inputs, the entering state and the adjoint flowing in
  {
    const int64_t xoff = (cp.row0 * p.H + cp.h) * DH, voff = (cp.row0 * p.H + cp.h) * NS;
    Slab<Q, DH, NT> U, G;
    Slab<Q, NS, NT> Bv, Cv;
    Slab<DH, NS, NT> Hs, Ls;
    float dv, av;
    U.load(p.u + xoff, (int64_t)p.H * DH, tid);
    G.load(p.dy + xoff, (int64_t)p.H * DH, tid);
    Bv.load(p.Bm + voff, (int64_t)p.H * NS, tid);
    Cv.load(p.Cm + voff, (int64_t)p.H * NS, tid);
    if (cp.c > 0) Hs.load(p.ckpt + (cp.bh * p.nC + cp.c - 1) * DH * NS, NS, tid);
    else if (p.h0 != nullptr) Hs.load(p.h0 + cp.bh * DH * NS, NS, tid);
    else Hs.zero();
    Ls.load(p.lamws + (cp.bh * p.nC + cp.c) * DH * NS, NS, tid);
    load_step<NS>(p, cp, tid, dv, av);
    U.store(sm.U, tid);
    G.store(sm.G, tid);
    Bv.store(sm.Bm, tid);
    Cv.store(sm.Cm, tid);
    Hs.store(sm.hin, tid);
    Ls.store(sm.lam, tid);
    step_scalars<NS, S::PN, NT>(dv, av, sm.del, sm.cd, sm.a, &sm.fac, sm.E, sm.m31, sm.ECt, sm.BEi, sm.Cm, sm.Bm, tid);
  }
  __syncthreads();
  // ---- B1: G2 = dY U^T, GH = dY h_in, UL = U lam (MFMA blocks: G2's four,
  //          then GH and UL, 2 NBN each); tr partials; W of a steep chunk
  constexpr int NBN = NS / 16;
  for (int blk = w; blk < 4 + 4 * NBN; blk += NW) {
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    if (blk < 4) {
      const int t0 = 16 * (blk >> 1), s0 = 16 * (blk & 1);
      acc = mm16<DH>([&](int r, int k) { return sm.G[t0 + r][k]; }, [&](int k, int c) { return sm.U[s0 + c][k]; },
                     lane, acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.G2[t0 + 4 * (lane >> 4) + r][s0 + (lane & 15)] = acc[r];
      continue;
    }
    const int kind = (blk - 4) / (2 * NBN), rem = (blk - 4) % (2 * NBN);
    const int t0 = 16 * (rem / NBN), n0 = 16 * (rem % NBN);
    if (kind == 0) {
      acc = mm16<DH>([&](int r, int k) { return sm.G[t0 + r][k]; },
                     [&](int k, int c) { return sm.hin[k][n0 + c]; }, lane, acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.GH[t0 + 4 * (lane >> 4) + r][n0 + (lane & 15)] = acc[r];
    } else {
      acc = mm16<DH>([&](int r, int k) { return sm.U[t0 + r][k]; },
                     [&](int k, int c) { return sm.lam[k][n0 + c]; }, lane, acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.UL[t0 + 4 * (lane >> 4) + r][n0 + (lane & 15)] = acc[r];
    }
  }
  {
    // tr[n] = sum_d lam o h_in: thread (part, n) sums d = part, part + P, ...
    constexpr int P = NT / NS;
    const int n = tid % NS, part = tid / NS;
    float s = 0.f;
#pragma unroll
    for (int d = part; d < DH; d += P) s += sm.lam[d][n] * sm.hin[d][n];
    sm.trp[part][n] = s;
  }
  const bool fast = __builtin_amdgcn_readfirstlane(__float_as_int(sm.fac.fast)) != 0;
  if (!fast) form_w<NS, S::PN, S::PQ, NT>(sm.W, sm.Cm, sm.Bm, sm.cd, sm.a, tid);
  __syncthreads();
  if (tid < NS) {
    float s = 0.f;
#pragma unroll
    for (int part = 0; part < NT / NS; ++part) s += sm.trp[part][tid];
    sm.tr[tid] = s;
  }
  // ---- B2: the masked sums over s and t (and W of a factored chunk)
  masked_sums<NS, NT, NW, true>(sm, fast, tid, w, lane);
  __syncthreads();
  // ---- C: du = diag(delta) (W^T dY + (B o m31) lam^T) (MFMA)
  constexpr int NBD = DH / 16;
  for (int blk = w; blk < 2 * NBD; blk += NW) {
    const int s0 = 16 * (blk / NBD), d0 = 16 * (blk % NBD);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16<Q>([&](int r, int k) { return sm.W[k][s0 + r]; }, [&](int k, int c) { return sm.G[k][d0 + c]; }, lane,
                  acc);
    acc = mm16<NS>([&](int r, int k) { return sm.Bm[s0 + r][k] * sm.m31[s0 + r][k]; },
                   [&](int k, int c) { return sm.lam[d0 + c][k]; }, lane, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int s = s0 + 4 * (lane >> 4) + r;
      rr::st(p.du, ((cp.row0 + s) * p.H + cp.h) * DH + d0 + (lane & 15), sm.del[s] * acc[r]);
    }
  }
  grad_epilogue<NS, NT, NW>(p, sm, cp, tid, w, lane);
}

// ------------------------------------------------------------------ wide states
// Dh 128 (and N 64): the chunk's state does not fit the LDS whole, so the
// output and gradient kernels stream it in blocks of kDB rows of d, staged
// through registers one block ahead.  Everything indexed by n (B, C, the
// decays, W, and the gradient's GH, UL, ZF, ZW, dC2) stays resident; the sums
// over d (Y's state term per block; the gradient's G2 = dY U^T, GH = dY h_in,
// UL = U lam and tr) accumulate in MFMA accumulators across the blocks, and du
// is formed block by block.
constexpr int kDB = 32;                   // rows of d per streamed block
constexpr int kStreamOutThreads = 256;
constexpr int kStreamGradThreads = 1024, kStreamGradWaves = kStreamGradThreads / 64;

template <int NS>
struct alignas(16) OutStreamSmem {
  static constexpr int PN = NS + 4, PQ = Q + 4, PB = kDB + 4;
  float Bm[Q][PN], Cm[Q][PN], E[Q][PN], ECt[Q][PN], BEi[Q][PN];
  float W[Q][PQ];
  float U[Q][PB];      // u of the block [s][d]
  float hin[kDB][PN];  // the entering state's rows of the block
  float del[Q], cd[Q], a[NS];
  Factor fac;
};

// The state entering chunk c, rows db * kDB .. + kDB - 1 (checkpoint c - 1,
// h0 or zero), into a slab.
template <int DH, int NS, int NT, typename InT>
__device__ __forceinline__ void load_hin_rows(Slab<kDB, NS, NT>& hs, const DenseArgsT<InT>& p, const ChunkPos& cp,
                                              int db, int tid) {
  if (cp.c > 0) hs.load(p.ckpt + (cp.bh * p.nC + cp.c - 1) * DH * NS + db * kDB * NS, NS, tid);
  else if (p.h0 != nullptr) hs.load(p.h0 + cp.bh * DH * NS + db * kDB * NS, NS, tid);
  else hs.zero();
}

template <typename InT, int DH, int NS>
__global__ __launch_bounds__(kStreamOutThreads) void dense_out_stream_kernel(DenseArgsT<InT> p) {
  constexpr int NT = kStreamOutThreads, NDB = DH / kDB;
  using S = OutStreamSmem<NS>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkPos cp = chunk_pos(p);
  const int64_t xoff = (cp.row0 * p.H + cp.h) * DH, voff = (cp.row0 * p.H + cp.h) * NS;
  Slab<Q, NS, NT> Bv, Cv;
  Slab<Q, kDB, NT> U;
  Slab<kDB, NS, NT> Hs;
  float dv, av;
  Bv.load(p.Bm + voff, (int64_t)p.H * NS, tid);
  Cv.load(p.Cm + voff, (int64_t)p.H * NS, tid);
  U.load(p.u + xoff, (int64_t)p.H * DH, tid);
  load_hin_rows<DH, NS, NT>(Hs, p, cp, 0, tid);
  load_step<NS>(p, cp, tid, dv, av);
  Bv.store(sm.Bm, tid);
  Cv.store(sm.Cm, tid);
  step_scalars<NS, S::PN, NT>(dv, av, sm.del, sm.cd, sm.a, &sm.fac, sm.E, nullptr, sm.ECt, sm.BEi, sm.Cm, sm.Bm, tid);
  __syncthreads();
  if (__builtin_amdgcn_readfirstlane(__float_as_int(sm.fac.fast)) != 0)
    form_w_block<NS, S::PN, S::PQ>(sm.W, sm.ECt, sm.BEi, 16 * (w >> 1), 16 * (w & 1), lane);
  else
    form_w<NS, S::PN, S::PQ, NT>(sm.W, sm.Cm, sm.Bm, sm.cd, sm.a, tid);
  for (int db = 0; db < NDB; ++db) {
    U.store(sm.U, tid);
    Hs.store(sm.hin, tid);
    __syncthreads();   // (also: W, for the first block)
    if (db + 1 < NDB) {   // the next block's loads, in flight during this one
      U.load(p.u + xoff + (db + 1) * kDB, (int64_t)p.H * DH, tid);
      load_hin_rows<DH, NS, NT>(Hs, p, cp, db + 1, tid);
    }
    // Y[t][d] = sum_s W[t][s] delta_s U[s][d] + sum_n C[t][n] E[t][n] hin[d][n]:
    // wave w, block (t0, d0) = (16 (w >> 1), 16 (w & 1)) of the kDB rows
    {
      const int t0 = 16 * (w >> 1), d0 = 16 * (w & 1);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      acc = mm16<Q>([&](int r, int k) { return sm.W[t0 + r][k] * sm.del[k]; },
                    [&](int k, int c) { return sm.U[k][d0 + c]; }, lane, acc);
      acc = mm16<NS>([&](int r, int k) { return sm.Cm[t0 + r][k] * sm.E[t0 + r][k]; },
                     [&](int k, int c) { return sm.hin[d0 + c][k]; }, lane, acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + 4 * (lane >> 4) + r;
        p.y[((cp.row0 + t) * p.H + cp.h) * DH + db * kDB + d0 + (lane & 15)] = acc[r];
      }
    }
    __syncthreads();   // the next block's stores overwrite U and hin
  }
}

template <int NS>
struct alignas(16) GradStreamSmem {
  static constexpr int PN = NS + 4, PQ = Q + 4, PB = kDB + 4;
  float Bm[Q][PN], Cm[Q][PN], E[Q][PN], m31[Q][PN], ECt[Q][PN], BEi[Q][PN];
  float G2[Q][PQ], W[Q][PQ];
  float GH[Q][PN], UL[Q][PN], ZF[Q][PN], ZW[Q][PN], dC2[Q][PN];
  float U[Q][PB], G[Q][PB];         // u, dY of the block [t][d]
  float hin[kDB][PN], lam[kDB][PN];  // the entering state's and the adjoint's rows of the block
  float del[Q], cd[Q], a[NS], trp[kStreamGradThreads / NS][NS], tr[NS];
  float ddp[kStreamGradWaves][2][Q];
  Factor fac;
};

template <typename InT, int DH, int NS>
__global__ __launch_bounds__(kStreamGradThreads) void dense_grad_stream_kernel(DenseArgsT<InT> p) {
  constexpr int NT = kStreamGradThreads, NW = kStreamGradWaves, NDB = DH / kDB, NBN = NS / 16;
  constexpr int NACC = 4 + 4 * NBN;   // accumulated blocks: G2 (4), GH (2 NBN), UL (2 NBN)
  static_assert(NACC <= 2 * NW, "two accumulated blocks per wave at most");
  using S = GradStreamSmem<NS>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkPos cp = chunk_pos(p);
  const int64_t xoff = (cp.row0 * p.H + cp.h) * DH, voff = (cp.row0 * p.H + cp.h) * NS;
  const int64_t soff = (cp.bh * p.nC + cp.c) * DH * NS;   // this chunk's adjoint slot
  Slab<Q, NS, NT> Bv, Cv;
  Slab<Q, kDB, NT> Us, Gs;
  Slab<kDB, NS, NT> Hs, Ls;
  float dv, av;
  Bv.load(p.Bm + voff, (int64_t)p.H * NS, tid);
  Cv.load(p.Cm + voff, (int64_t)p.H * NS, tid);
  Us.load(p.u + xoff, (int64_t)p.H * DH, tid);
  Gs.load(p.dy + xoff, (int64_t)p.H * DH, tid);
  load_hin_rows<DH, NS, NT>(Hs, p, cp, 0, tid);
  Ls.load(p.lamws + soff, NS, tid);
  load_step<NS>(p, cp, tid, dv, av);
  Bv.store(sm.Bm, tid);
  Cv.store(sm.Cm, tid);
  step_scalars<NS, S::PN, NT>(dv, av, sm.del, sm.cd, sm.a, &sm.fac, sm.E, sm.m31, sm.ECt, sm.BEi, sm.Cm, sm.Bm, tid);
  __syncthreads();
  const bool fast = __builtin_amdgcn_readfirstlane(__float_as_int(sm.fac.fast)) != 0;
  // W first: du, formed block by block, needs it
  if (fast) {
    if (w < 4) form_w_block<NS, S::PN, S::PQ>(sm.W, sm.ECt, sm.BEi, 16 * (w >> 1), 16 * (w & 1), lane);
  } else {
    form_w<NS, S::PN, S::PQ, NT>(sm.W, sm.Cm, sm.Bm, sm.cd, sm.a, tid);
  }
  // accumulated blocks of this wave: b = w and w + NW (b < NACC); du blocks of
  // a d-block (2 row blocks s x 2 column blocks d): waves NW - 4 .. NW - 1
  f32x4_t acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  float trs = 0.f;   // this thread's share of tr[n], n = tid % NS (NT is a multiple of NS)
  for (int db = 0; db < NDB; ++db) {
    Us.store(sm.U, tid);
    Gs.store(sm.G, tid);
    Hs.store(sm.hin, tid);
    Ls.store(sm.lam, tid);
    __syncthreads();   // (also: W, for the first block)
    if (db + 1 < NDB) {
      Us.load(p.u + xoff + (db + 1) * kDB, (int64_t)p.H * DH, tid);
      Gs.load(p.dy + xoff + (db + 1) * kDB, (int64_t)p.H * DH, tid);
      load_hin_rows<DH, NS, NT>(Hs, p, cp, db + 1, tid);
      Ls.load(p.lamws + soff + (db + 1) * kDB * NS, NS, tid);
    }
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int b = w + NW * m;
      if (b >= NACC) continue;
      if (b < 4) {   // G2[t][s] += sum_d dY[t][d] U[s][d]
        const int t0 = 16 * (b >> 1), s0 = 16 * (b & 1);
        acc[m] = mm16<kDB>([&](int r, int k) { return sm.G[t0 + r][k]; },
                           [&](int k, int c) { return sm.U[s0 + c][k]; }, lane, acc[m]);
      } else {
        const int kind = (b - 4) / (2 * NBN), rem = (b - 4) % (2 * NBN);
        const int t0 = 16 * (rem / NBN), n0 = 16 * (rem % NBN);
        if (kind == 0)   // GH[t][n] += sum_d dY[t][d] h_in[d][n]
          acc[m] = mm16<kDB>([&](int r, int k) { return sm.G[t0 + r][k]; },
                             [&](int k, int c) { return sm.hin[k][n0 + c]; }, lane, acc[m]);
        else             // UL[s][n] += sum_d U[s][d] lam[d][n]
          acc[m] = mm16<kDB>([&](int r, int k) { return sm.U[t0 + r][k]; },
                             [&](int k, int c) { return sm.lam[k][n0 + c]; }, lane, acc[m]);
      }
    }
    if (w >= NW - 4) {
      // du[s][d] = delta_s (sum_t W[t][s] dY[t][d] + sum_n B[s][n] m31[s][n] lam[d][n])
      const int v = w - (NW - 4), s0 = 16 * (v >> 1), d0 = 16 * (v & 1);
      f32x4_t du = {0.f, 0.f, 0.f, 0.f};
      du = mm16<Q>([&](int r, int k) { return sm.W[k][s0 + r]; }, [&](int k, int c) { return sm.G[k][d0 + c]; },
                   lane, du);
      du = mm16<NS>([&](int r, int k) { return sm.Bm[s0 + r][k] * sm.m31[s0 + r][k]; },
                    [&](int k, int c) { return sm.lam[d0 + c][k]; }, lane, du);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = s0 + 4 * (lane >> 4) + r;
        rr::st(p.du, ((cp.row0 + s) * p.H + cp.h) * DH + db * kDB + d0 + (lane & 15), sm.del[s] * du[r]);
      }
    }
#pragma unroll
    for (int j = 0; j < (kDB * NS + NT - 1) / NT; ++j) {   // tr partials (elements in column tid % NS)
      const int i = tid + NT * j;
      if (kDB * NS % NT == 0 || i < kDB * NS) trs += sm.lam[i / NS][i % NS] * sm.hin[i / NS][i % NS];
    }
    __syncthreads();   // the next block's stores overwrite the staging
  }
  // the accumulated blocks into LDS; tr
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const int b = w + NW * m;
    if (b >= NACC) continue;
    if (b < 4) {
      const int t0 = 16 * (b >> 1), s0 = 16 * (b & 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.G2[t0 + 4 * (lane >> 4) + r][s0 + (lane & 15)] = acc[m][r];
    } else {
      const int kind = (b - 4) / (2 * NBN), rem = (b - 4) % (2 * NBN);
      const int t0 = 16 * (rem / NBN), n0 = 16 * (rem % NBN);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        if (kind == 0) sm.GH[t0 + 4 * (lane >> 4) + r][n0 + (lane & 15)] = acc[m][r];
        else sm.UL[t0 + 4 * (lane >> 4) + r][n0 + (lane & 15)] = acc[m][r];
      }
    }
  }
  sm.trp[tid / NS][tid % NS] = trs;
  __syncthreads();
  if (tid < NS) {
    float t = 0.f;
#pragma unroll
    for (int part = 0; part < NT / NS; ++part) t += sm.trp[part][tid];
    sm.tr[tid] = t;
  }
  masked_sums<NS, NT, NW, false>(sm, fast, tid, w, lane);
  __syncthreads();
  grad_epilogue<NS, NT, NW>(p, sm, cp, tid, w, lane);
}

template <typename InT, int DH, int NS>
int launch(const rr::DenseArgs& a, int what, hipStream_t s) {
  DenseArgsT<InT> p;
  p.u = static_cast<const InT*>(a.u);
  p.delta = static_cast<const InT*>(a.delta);
  p.Bm = static_cast<const InT*>(a.Bm);
  p.Cm = static_cast<const InT*>(a.Cm);
  p.A = a.A;
  p.a_sh = a.a_sh;
  p.a_sn = a.a_sn;
  p.h0 = a.h0;
  p.ckpt = a.ckpt;
  p.lamws = a.lamws;
  p.dy = a.dy;
  p.y = a.y;
  p.du = static_cast<InT*>(a.du);
  p.ddelta = static_cast<InT*>(a.ddelta);
  p.dB = static_cast<InT*>(a.dB);
  p.dC = static_cast<InT*>(a.dC);
  p.gA_part = a.gA_part;
  p.mapE = a.mapE;
  p.mapP = a.mapP;
  p.B = a.B; p.L = a.L; p.H = a.H; p.DH = a.DH; p.NS = a.NS; p.nC = a.nC;
  const dim3 grid((unsigned)((int64_t)a.B * a.H * a.nC)), blk(256);
  constexpr bool kStream = DH > 64 || NS > 32;   // the state streamed in blocks of d (wide states)
  switch (what) {
    case rr::kDenseMapsFwd: hipLaunchKernelGGL((dense_map_kernel<InT, DH, NS, false>), grid, blk, 0, s, p); break;
    case rr::kDenseMapsBwd: hipLaunchKernelGGL((dense_map_kernel<InT, DH, NS, true>), grid, blk, 0, s, p); break;
    case rr::kDenseOut:
      if constexpr (kStream)
        hipLaunchKernelGGL((dense_out_stream_kernel<InT, DH, NS>), grid, dim3(kStreamOutThreads), 0, s, p);
      else
        hipLaunchKernelGGL((dense_out_kernel<InT, DH, NS>), grid, dim3(kOutThreads), 0, s, p);
      break;
    default:
      if constexpr (kStream)
        hipLaunchKernelGGL((dense_grad_stream_kernel<InT, DH, NS>), grid, dim3(kStreamGradThreads), 0, s, p);
      else
        hipLaunchKernelGGL((dense_grad_kernel<InT, DH, NS>), grid, dim3(kGradThreads), 0, s, p);
      break;
  }
  return rr::check_launch(what == rr::kDenseOut ? "ssd dense forward" : what == rr::kDenseGrad ? "ssd dense backward"
                                                                                               : "ssd dense chunk maps");
}

template <typename InT>
int launch_shape(const rr::DenseArgs& a, int what, hipStream_t s) {
  switch (a.DH * 1000 + a.NS) {
    case 32016: return launch<InT, 32, 16>(a, what, s);
    case 32032: return launch<InT, 32, 32>(a, what, s);
    case 64016: return launch<InT, 64, 16>(a, what, s);
    case 64032: return launch<InT, 64, 32>(a, what, s);
    case 64064: return launch<InT, 64, 64>(a, what, s);
    case 128016: return launch<InT, 128, 16>(a, what, s);
    case 128032: return launch<InT, 128, 32>(a, what, s);
    case 128064: return launch<InT, 128, 64>(a, what, s);
    default: return rr::fail(RR_EUNSUPPORTED, "ssd dense: unsupported (Dh, N)");
  }
}

}  // namespace

namespace rr {

bool ssd_dense_supported(int64_t T, int64_t Dh, int64_t N, int64_t B, int64_t H, int64_t nC) {
  return T == Q && B * H * nC < ((int64_t)1 << 31) &&
         (((Dh == 32 || Dh == 64) && (N == 16 || N == 32)) || (Dh == 64 && N == 64) ||
          (Dh == 128 && (N == 16 || N == 32 || N == 64)));
}

int ssd_dense_launch(const DenseArgs& a, int dtype, int what, hipStream_t s) {
  switch (dtype) {
    case RR_F32: return launch_shape<float>(a, what, s);
    case RR_BF16: return launch_shape<bf16>(a, what, s);
    case RR_F16: return launch_shape<f16>(a, what, s);
    default: return fail(RR_EINVAL, "ssd dense: unsupported dtype");
  }
}

int dense_compose(const float* mapE, const float* mapP, const float* x0, float* out, float* xlast, int64_t B,
                  int64_t H, int64_t Dh, int64_t N, int64_t nC, bool bwd, bool gla, hipStream_t s) {
  const int64_t total = B * H * Dh * N;
  const dim3 grid((unsigned)((total + 255) / 256)), blk(256);
  const int dl = (int)Dh, ns = (int)N, nc = (int)nC;
  if (bwd && gla)
    hipLaunchKernelGGL((dense_compose_kernel<true, true>), grid, blk, 0, s, mapE, mapP, x0, out, xlast, total, dl, ns, nc);
  else if (bwd)
    hipLaunchKernelGGL((dense_compose_kernel<true, false>), grid, blk, 0, s, mapE, mapP, x0, out, xlast, total, dl, ns, nc);
  else if (gla)
    hipLaunchKernelGGL((dense_compose_kernel<false, true>), grid, blk, 0, s, mapE, mapP, x0, out, xlast, total, dl, ns, nc);
  else
    hipLaunchKernelGGL((dense_compose_kernel<false, false>), grid, blk, 0, s, mapE, mapP, x0, out, xlast, total, dl, ns, nc);
  return check_launch(bwd ? "dense backward adjoints" : "dense forward states");
}

}  // namespace rr
