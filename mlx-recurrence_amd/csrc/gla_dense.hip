// gla_dense.hip — GLA (reference gla.py:78-100, adjoint gla.py:184-236) for
// fp32 / fp16 inputs in chunked form on the fp32 MFMA, chunks of 32 steps
// (bf16 inputs take the chunked kernels of rr_chunked.h / chunked_bwd.hip,
// whose operands are exact in bf16).
//
// Per chunk of one (batch, head), with the state h[j, i] (j value index, i key
// index), gates g_t, M[t, s] = g_{s+1} ... g_t (t >= s; 0 else), formed as
// running products (so gates of either sign, and zero, are exact),
// gam_t = g_0 ... g_t, m31_s = M[31, s], h_in the state entering the chunk
// and lam the adjoint of its last state flowing in from later chunks:
//   chunk maps: forward  S  = V^T diag(m31) K;  the state after the chunk is gam_31 h_in + S
//               backward S' = dY^T diag(gam) Q; the adjoint handed back is gam_31 lam + S'
//   Y  = (M o Q K^T) V + diag(gam) Q h_in^T
//   with CB = Q K^T, G2 = dY V^T, GH = dY h_in, UL = V lam, P = M o CB, MG = M o G2:
//   dq = diag(gam) GH + MG K
//   dk = MG^T Q + diag(m31) UL
//   dv = P^T dY + diag(m31) K lam^T
//   dg_t = sum_{j,i} lam_t h_{t-1}
//        = sum_{t'} M[t', t] (E Mh + X gam_{t-1})[t', t] + m31_t (P_t + gam_{t-1} tr),
//     E = CB o G2, Mh[s, t] = M[t-1, s] (s < t; 0 else), X = rowsum(GH o Q),
//     Y = rowsum(UL o K), P_t = sum_s Mh[s, t] Y_s, tr = sum lam o h_in
//   (lam_t and h_{t-1} expand through M[t', t] and M[t-1, s], so no gate is
//   ever divided by; derived from the per-step adjoint and checked in float64
//   against the oracle before this code).
// Three kernels per pass, as for SSD (ssd_dense.hip): chunk maps, the walk
// over them (rr_dense.h), every chunk's outputs or gradients.
#include "rr_common.h"
#include "rr_dense.h"
#include "rr_internal.h"
#include "rr_mfma.h"

namespace {

using namespace rr::dense;

template <typename InT>
struct GlaArgsT {
  const InT* q;
  const InT* k;
  const InT* v;
  const InT* g;
  const float* h0;      // [B,H,D,D] as the reference's [i][j], or null
  const float* ckpt;    // [B,H,nC,D,D] as [j][i]: the state after each chunk
  const float* lamws;   // [B,H,nC,D,D] as [j][i]: the adjoint flowing into each chunk's end
  const float* dy;      // [B,L,H,D]
  float* y;
  InT* dq;
  InT* dk;
  InT* dv;
  InT* dg;
  float* mapE;          // [B,H,nC,D,D] as [j][i]
  float* mapP;          // [B,H,nC,D]: gam_31 in every column
  int B, L, H, nC;
};

// Decays of the chunk from its gates (g in LDS): M[t][s] by the first 32
// lanes (lane s walks column s), then gam, gam_{t-1} and m31.  Leaves with a
// barrier.
template <int PQ>
__device__ __forceinline__ void gate_products(const float* g, float (*M)[PQ], float* gam, float* gm1, float* m31,
                                              int tid) {
  if (tid < Q) {
    const int s = tid;
    float x = 1.f;
#pragma unroll 8
    for (int t = 0; t < Q; ++t) {
      if (t > s) x *= g[t];
      M[t][s] = t >= s ? x : 0.f;
    }
  }
  __syncthreads();
  if (tid < Q) {
    gam[tid] = g[0] * M[tid][0];
    gm1[tid] = tid == 0 ? 1.f : g[0] * M[tid - 1][0];
    m31[tid] = M[Q - 1][tid];
  }
  __syncthreads();
}

// The state entering chunk c, as [j][i]: checkpoint c - 1, else h0 (stored
// [i][j]), else zero.
template <int D, int NT, typename InT>
__device__ __forceinline__ void load_entering(Slab<D, D, NT>& hs, const GlaArgsT<InT>& p, const ChunkPos& cp,
                                              int tid) {
  if (cp.c > 0) hs.load(p.ckpt + (cp.bh * p.nC + cp.c - 1) * D * D, D, tid);
  else if (p.h0 != nullptr) hs.load_t(p.h0 + cp.bh * D * D, D, tid);
  else hs.zero();
}

// ------------------------------------------------------------------ chunk maps
// Forward: S[j][i] = sum_s v_s[j] m31_s k_s[i]; backward: S'[j][i] =
// sum_t dY_t[j] gam_t q_t[i]; P = gam_31 in every column.
template <int D>
struct alignas(16) GlaMapSmem {
  static constexpr int PD = D + 4;
  float X[Q][PD];   // v (forward) or dY (backward)
  float Y[Q][PD];   // k (forward) or q (backward)
  float g[Q], w[Q], tot;
};

// Workgroup size of the map and output kernels: eight waves (the chunk's
// 16 x 16 output blocks spread over more waves).
constexpr int kGlaSmallThreads = 512, kGlaSmallWaves = kGlaSmallThreads / 64;

template <typename InT, int D, bool BWD>
__global__ __launch_bounds__(kGlaSmallThreads) void gla_map_kernel(GlaArgsT<InT> p) {
  constexpr int NT = kGlaSmallThreads, NW = kGlaSmallWaves;
  __shared__ GlaMapSmem<D> sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkPos cp = chunk_pos(p.H, p.L, p.nC);
  const int64_t off = (cp.row0 * p.H + cp.h) * D, stride = (int64_t)p.H * D;
  Slab<Q, D, NT> X, Y;
  if constexpr (BWD) {
    X.load(p.dy + off, stride, tid);
    Y.load(p.q + off, stride, tid);
  } else {
    X.load(p.v + off, stride, tid);
    Y.load(p.k + off, stride, tid);
  }
  const float gv = rr::ld(p.g, (cp.row0 + (tid & (Q - 1))) * p.H + cp.h);
  X.store(sm.X, tid);
  Y.store(sm.Y, tid);
  if (tid < Q) sm.g[tid] = gv;
  __syncthreads();
  if (tid < Q) {   // forward m31_t = g_{t+1} ... g_31; backward gam_t = g_0 ... g_t
    float x = 1.f;
    if constexpr (BWD) {
      for (int t = 0; t <= tid; ++t) x *= sm.g[t];
    } else {
      for (int t = tid + 1; t < Q; ++t) x *= sm.g[t];
    }
    sm.w[tid] = x;
    if (tid == (BWD ? Q - 1 : 0)) sm.tot = BWD ? x : sm.g[0] * x;   // gam_31
  }
  __syncthreads();
  constexpr int NB = D / 16;
  float* dst = p.mapE + (cp.bh * p.nC + cp.c) * D * D;
  for (int blk = w; blk < NB * NB; blk += NW) {
    const int j0 = 16 * (blk / NB), i0 = 16 * (blk % NB);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = mm16<Q>([&](int r, int k) { return sm.X[k][j0 + r]; },
                  [&](int k, int c) { return sm.w[k] * sm.Y[k][i0 + c]; }, lane, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(j0 + 4 * (lane >> 4) + r) * D + i0 + (lane & 15)] = acc[r];
  }
  if (tid < D) p.mapP[(cp.bh * p.nC + cp.c) * D + tid] = sm.tot;
}

// ------------------------------------------------------------------ forward y
template <int D>
struct alignas(16) GlaOutSmem {
  static constexpr int PD = D + 4, PQ = Q + 4;
  float Qm[Q][PD], K[Q][PD], V[Q][PD];
  float hin[D][PD];
  float M[Q][PQ], P[Q][PQ];
  float g[Q], gam[Q], gm1[Q], m31[Q];
};

template <typename InT, int D>
__global__ __launch_bounds__(kGlaSmallThreads) void gla_out_kernel(GlaArgsT<InT> p) {
  constexpr int NT = kGlaSmallThreads, NW = kGlaSmallWaves;
  using S = GlaOutSmem<D>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkPos cp = chunk_pos(p.H, p.L, p.nC);
  const int64_t off = (cp.row0 * p.H + cp.h) * D, stride = (int64_t)p.H * D;
  {
    Slab<Q, D, NT> Qs, Ks, Vs;
    Slab<D, D, NT> Hs;
    Qs.load(p.q + off, stride, tid);
    Ks.load(p.k + off, stride, tid);
    Vs.load(p.v + off, stride, tid);
    load_entering<D, NT>(Hs, p, cp, tid);
    const float gv = rr::ld(p.g, (cp.row0 + (tid & (Q - 1))) * p.H + cp.h);
    Qs.store(sm.Qm, tid);
    Ks.store(sm.K, tid);
    Vs.store(sm.V, tid);
    Hs.store(sm.hin, tid);
    if (tid < Q) sm.g[tid] = gv;
  }
  __syncthreads();
  gate_products<S::PQ>(sm.g, sm.M, sm.gam, sm.gm1, sm.m31, tid);
  if (w < 4) {
    // P = M o (Q K^T): wave w, block (w >> 1, w & 1) (the upper one is zero)
    const int t0 = 16 * (w >> 1), s0 = 16 * (w & 1);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    if (t0 >= s0)
      acc = mm16<D>([&](int r, int k) { return sm.Qm[t0 + r][k]; }, [&](int k, int c) { return sm.K[s0 + c][k]; },
                    lane, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * (lane >> 4) + r, s = s0 + (lane & 15);
      sm.P[t][s] = sm.M[t][s] * acc[r];
    }
  }
  __syncthreads();
  // Y[t][j] = sum_{s <= t} P[t][s] V[s][j] + gam_t sum_i Q[t][i] hin[j][i]
  constexpr int NB = D / 16;
  for (int blk = w; blk < 2 * NB; blk += NW) {
    const int t0 = 16 * (blk / NB), j0 = 16 * (blk % NB);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    const auto fp = [&](int r, int k) { return sm.P[t0 + r][k]; };
    const auto fv = [&](int k, int c) { return sm.V[k][j0 + c]; };
    acc = t0 == 0 ? mm16r<0, 16>(fp, fv, lane, acc) : mm16r<0, Q>(fp, fv, lane, acc);
    acc = mm16<D>([&](int r, int k) { return sm.gam[t0 + r] * sm.Qm[t0 + r][k]; },
                  [&](int k, int c) { return sm.hin[j0 + c][k]; }, lane, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * (lane >> 4) + r;
      p.y[((cp.row0 + t) * p.H + cp.h) * D + j0 + (lane & 15)] = acc[r];
    }
  }
}

// ------------------------------------------------------------------ backward
// Eight waves per chunk.  Phase B1 forms every product that reads v, h_in or
// lam into registers; after a barrier those inputs are dead and their LDS
// holds P, MG, E, GH and UL.  Waves 0-3 own the CB / G2 blocks, GH, dq and
// dk; waves 4-7 own UL, K lam^T (kept in registers into dv) and dv, and the
// dg column sums.
constexpr int kGlaGradThreads = 512;
template <int D>
struct alignas(16) GlaGradSmem {
  static constexpr int PD = D + 4, PQ = Q + 4;
  float Qm[Q][PD], K[Q][PD], G[Q][PD];
  union {
    struct {
      float V[Q][PD];
      float hin[D][PD];
      float lam[D][PD];
    } a;
    struct {
      float GH[Q][PD], UL[Q][PD];
      float P[Q][PQ], MG[Q][PQ], E[Q][PQ];
    } b;
  } u;
  float M[Q][PQ];
  float g[Q], gam[Q], gm1[Q], m31[Q];
  float Xp[4][Q], Yp[4][Q];   // per column-block row sums of GH o Q and UL o K
  float HpP[2][Q];            // per row-block column sums of M o (E Mh + X gam_{t-1})
  float trw[kGlaGradThreads / 64];
};

template <typename InT, int D>
__global__ __launch_bounds__(kGlaGradThreads) void gla_grad_kernel(GlaArgsT<InT> p) {
  constexpr int NT = kGlaGradThreads, NB = D / 16, NM = NB / 2;   // NM: blocks per wave of each 2 NB kind
  using S = GlaGradSmem<D>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l15 = lane & 15, l4 = lane >> 4;
  const ChunkPos cp = chunk_pos(p.H, p.L, p.nC);
  const int64_t off = (cp.row0 * p.H + cp.h) * D, stride = (int64_t)p.H * D;
  // ---- A: inputs, the entering state, the adjoint flowing in; the decays
  {
    Slab<Q, D, NT> Qs, Ks, Vs, Gs;
    Slab<D, D, NT> Hs, Ls;
    Qs.load(p.q + off, stride, tid);
    Ks.load(p.k + off, stride, tid);
    Vs.load(p.v + off, stride, tid);
    Gs.load(p.dy + off, stride, tid);
    load_entering<D, NT>(Hs, p, cp, tid);
    Ls.load(p.lamws + (cp.bh * p.nC + cp.c) * D * D, D, tid);
    const float gv = rr::ld(p.g, (cp.row0 + (tid & (Q - 1))) * p.H + cp.h);
    Qs.store(sm.Qm, tid);
    Ks.store(sm.K, tid);
    Vs.store(sm.u.a.V, tid);
    Gs.store(sm.G, tid);
    Hs.store(sm.u.a.hin, tid);
    Ls.store(sm.u.a.lam, tid);
    if (tid < Q) sm.g[tid] = gv;
  }
  __syncthreads();
  gate_products<S::PQ>(sm.g, sm.M, sm.gam, sm.gm1, sm.m31, tid);
  // ---- B1 (registers): waves 0-3: CB, G2 of block (w >> 1, w & 1) -> E, P, MG;
  //      GH blocks w + 4 m.  Waves 4-7 (v = w - 4): UL and K lam^T blocks v + 4 m.
  f32x4_t e4 = {0.f, 0.f, 0.f, 0.f}, p4 = e4, mg4 = e4;
  f32x4_t blk4[NM], kl4[NM];
  const int v = w - 4;
  if (w < 4) {
    const int t0 = 16 * (w >> 1), s0 = 16 * (w & 1);
    if (t0 >= s0) {
      f32x4_t cb = {0.f, 0.f, 0.f, 0.f}, g2 = cb;
      cb = mm16<D>([&](int r, int k) { return sm.Qm[t0 + r][k]; }, [&](int k, int c) { return sm.K[s0 + c][k]; },
                   lane, cb);
      g2 = mm16<D>([&](int r, int k) { return sm.G[t0 + r][k]; }, [&](int k, int c) { return sm.u.a.V[s0 + c][k]; },
                   lane, g2);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float m = sm.M[t0 + 4 * l4 + r][s0 + l15];
        e4[r] = cb[r] * g2[r];
        p4[r] = m * cb[r];
        mg4[r] = m * g2[r];
      }
    }
#pragma unroll
    for (int m = 0; m < NM; ++m) {   // GH[t][i] = sum_j dY[t][j] h_in[j][i]; X partials
      const int b = w + 4 * m, t0g = 16 * (b / NB), i0 = 16 * (b % NB);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      acc = mm16<D>([&](int r, int k) { return sm.G[t0g + r][k]; },
                    [&](int k, int c) { return sm.u.a.hin[k][i0 + c]; }, lane, acc);
      blk4[m] = acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0g + 4 * l4 + r;
        const float x = rr::row16_sum(acc[r] * sm.Qm[t][i0 + l15]);
        if (l15 == 0) sm.Xp[b % NB][t] = x;
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const int b = v + 4 * m, s0 = 16 * (b / NB), c0 = 16 * (b % NB);
      // UL[s][i] = sum_j V[s][j] lam[j][i]; Y partials
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      acc = mm16<D>([&](int r, int k) { return sm.u.a.V[s0 + r][k]; },
                    [&](int k, int c) { return sm.u.a.lam[k][c0 + c]; }, lane, acc);
      blk4[m] = acc;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = s0 + 4 * l4 + r;
        const float y = rr::row16_sum(acc[r] * sm.K[s][c0 + l15]);
        if (l15 == 0) sm.Yp[b % NB][s] = y;
      }
      // KL[s][j] = sum_i K[s][i] lam[j][i] (the diag(m31) K lam^T part of dv)
      f32x4_t kl = {0.f, 0.f, 0.f, 0.f};
      kl = mm16<D>([&](int r, int k) { return sm.K[s0 + r][k]; },
                   [&](int k, int c) { return sm.u.a.lam[c0 + c][k]; }, lane, kl);
      kl4[m] = kl;
    }
  }
  {
    // tr = sum lam o h_in: per-wave partials
    float t = 0.f;
#pragma unroll
    for (int j = 0; j < D * D / NT; ++j) {
      const int i = tid + NT * j;
      t += sm.u.a.lam[i / D][i % D] * sm.u.a.hin[i / D][i % D];
    }
    t = rr::wave_sum(t);
    if (lane == 0) sm.trw[w] = t;
  }
  __syncthreads();   // v, h_in and lam are dead from here on
  if (w < 4) {
    const int t0 = 16 * (w >> 1), s0 = 16 * (w & 1);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * l4 + r, s = s0 + l15;
      sm.u.b.E[t][s] = e4[r];
      sm.u.b.P[t][s] = p4[r];
      sm.u.b.MG[t][s] = mg4[r];
    }
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const int b = w + 4 * m, t0g = 16 * (b / NB), i0 = 16 * (b % NB);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.u.b.GH[t0g + 4 * l4 + r][i0 + l15] = blk4[m][r];
    }
  } else {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const int b = v + 4 * m, s0 = 16 * (b / NB), c0 = 16 * (b % NB);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.u.b.UL[s0 + 4 * l4 + r][c0 + l15] = blk4[m][r];
    }
  }
  __syncthreads();
  // ---- B2: waves 0-3: dq, dk blocks w + 4 m.  Waves 4-7: dv blocks v + 4 m;
  //      waves 4-6: the dg column sums of W2 = E Mh blocks (0,0), (1,0), (1,1).
  if (w < 4) {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const int b = w + 4 * m, r0 = 16 * (b / NB), i0 = 16 * (b % NB);
      {
        // dq[t][i] = gam_t GH[t][i] + sum_{s <= t} MG[t][s] K[s][i]
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        const auto fa = [&](int r, int k) { return sm.u.b.MG[r0 + r][k]; };
        const auto fb = [&](int k, int c) { return sm.K[k][i0 + c]; };
        acc = r0 == 0 ? mm16r<0, 16>(fa, fb, lane, acc) : mm16r<0, Q>(fa, fb, lane, acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = r0 + 4 * l4 + r;
          rr::st(p.dq, ((cp.row0 + t) * p.H + cp.h) * D + i0 + l15, acc[r] + sm.gam[t] * sm.u.b.GH[t][i0 + l15]);
        }
      }
      {
        // dk[s][i] = sum_{t >= s} MG[t][s] Q[t][i] + m31_s UL[s][i]
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        const auto fa = [&](int r, int k) { return sm.u.b.MG[k][r0 + r]; };
        const auto fb = [&](int k, int c) { return sm.Qm[k][i0 + c]; };
        acc = r0 == 0 ? mm16r<0, Q>(fa, fb, lane, acc) : mm16r<16, Q>(fa, fb, lane, acc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = r0 + 4 * l4 + r;
          rr::st(p.dk, ((cp.row0 + s) * p.H + cp.h) * D + i0 + l15, acc[r] + sm.m31[s] * sm.u.b.UL[s][i0 + l15]);
        }
      }
    }
  } else {
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      // dv[s][j] = sum_{t >= s} P[t][s] dY[t][j] + m31_s KL[s][j]
      const int b = v + 4 * m, s0 = 16 * (b / NB), j0 = 16 * (b % NB);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      const auto fa = [&](int r, int k) { return sm.u.b.P[k][s0 + r]; };
      const auto fb = [&](int k, int c) { return sm.G[k][j0 + c]; };
      acc = s0 == 0 ? mm16r<0, Q>(fa, fb, lane, acc) : mm16r<16, Q>(fa, fb, lane, acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = s0 + 4 * l4 + r;
        rr::st(p.dv, ((cp.row0 + s) * p.H + cp.h) * D + j0 + l15, acc[r] + sm.m31[s] * kl4[m][r]);
      }
    }
    if (v < 3) {
      // W2[t'][t] = sum_{s < t} E[t'][s] M[t-1][s]; column sums over t' of
      // M[t'][t] (W2 + X[t'] gam_{t-1}) for rows tp0 .. tp0 + 15
      const int tp0 = v == 0 ? 0 : 16, t0 = v == 2 ? 16 : 0;
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      const auto fa = [&](int r, int k) { return sm.u.b.E[tp0 + r][k]; };
      const auto fb = [&](int k, int c) {
        const int t = t0 + c;
        return k < t ? sm.M[t - 1][k] : 0.f;
      };
      acc = t0 == 0 ? mm16r<0, 16>(fa, fb, lane, acc) : mm16r<0, Q>(fa, fb, lane, acc);
      const int t = t0 + l15;
      float cs = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tp = tp0 + 4 * l4 + r;
        float x = 0.f;
#pragma unroll
        for (int ib = 0; ib < NB; ++ib) x += sm.Xp[ib][tp];
        cs += sm.M[tp][t] * (acc[r] + x * sm.gm1[t]);
      }
      cs += __shfl_xor(cs, 16);
      cs += __shfl_xor(cs, 32);
      if (l4 == 0) sm.HpP[tp0 / 16][t] = cs;
    }
  }
  __syncthreads();
  // ---- C: dg_t = the column sums + m31_t (P_t + gam_{t-1} tr),
  //      P_t = sum_{s < t} M[t-1][s] Y_s
  if (tid < Q) {
    const int t = tid;
    float tr = 0.f;
#pragma unroll
    for (int ww = 0; ww < NT / 64; ++ww) tr += sm.trw[ww];
    float pt = 0.f;
    for (int s = 0; s < t; ++s) {
      float y = 0.f;
#pragma unroll
      for (int ib = 0; ib < NB; ++ib) y += sm.Yp[ib][s];
      pt += sm.M[t - 1][s] * y;
    }
    const float hp = (t < 16 ? sm.HpP[0][t] : 0.f) + sm.HpP[1][t];
    rr::st(p.dg, (cp.row0 + t) * p.H + cp.h, hp + sm.m31[t] * (pt + sm.gm1[t] * tr));
  }
}

// ------------------------------------------------------------------ wide states
// Dh 128: the 128 x 128 state is streamed in blocks of kJB rows of j (the value
// index), staged through registers one block ahead; q, k and the decays stay
// resident.  The forward forms Y per block; the backward accumulates the sums
// over j (G2 = dY V^T, GH = dY h_in, UL = V lam, tr) in MFMA accumulators
// across the blocks and forms dv (with K lam^T) per block; dq, dk and dg follow
// the loop as in the resident kernel (E and MG formed from CB, G2 and M).
constexpr int kJB = 32;
constexpr int kGlaStreamOutThreads = 256;
constexpr int kGlaStreamGradThreads = 1024, kGlaStreamGradWaves = kGlaStreamGradThreads / 64;

// Rows j0 .. j0 + kJB - 1 of the state entering chunk c, as [j][i].
template <int D, int NT, typename InT>
__device__ __forceinline__ void load_entering_rows(Slab<kJB, D, NT>& hs, const GlaArgsT<InT>& p, const ChunkPos& cp,
                                                   int j0, int tid) {
  if (cp.c > 0) hs.load(p.ckpt + (cp.bh * p.nC + cp.c - 1) * D * D + (int64_t)j0 * D, D, tid);
  else if (p.h0 != nullptr) hs.load_t(p.h0 + cp.bh * D * D + j0, D, tid);   // h0 is [i][j]
  else hs.zero();
}

template <int D>
struct alignas(16) GlaOutStreamSmem {
  static constexpr int PD = D + 4, PQ = Q + 4, PB = kJB + 4;
  float Qm[Q][PD], K[Q][PD];
  float M[Q][PQ], P[Q][PQ];
  float V[Q][PB];       // v of the block [s][j]
  float hin[kJB][PD];   // the entering state's rows of the block [j][i]
  float g[Q], gam[Q], gm1[Q], m31[Q];
};

template <typename InT, int D>
__global__ __launch_bounds__(kGlaStreamOutThreads) void gla_out_stream_kernel(GlaArgsT<InT> p) {
  constexpr int NT = kGlaStreamOutThreads, NJB = D / kJB;
  using S = GlaOutStreamSmem<D>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkPos cp = chunk_pos(p.H, p.L, p.nC);
  const int64_t off = (cp.row0 * p.H + cp.h) * D, stride = (int64_t)p.H * D;
  Slab<Q, kJB, NT> Vs;
  Slab<kJB, D, NT> Hs;
  {
    Slab<Q, D, NT> Qs, Ks;
    Qs.load(p.q + off, stride, tid);
    Ks.load(p.k + off, stride, tid);
    Vs.load(p.v + off, stride, tid);
    load_entering_rows<D, NT>(Hs, p, cp, 0, tid);
    const float gv = rr::ld(p.g, (cp.row0 + (tid & (Q - 1))) * p.H + cp.h);
    Qs.store(sm.Qm, tid);
    Ks.store(sm.K, tid);
    if (tid < Q) sm.g[tid] = gv;
  }
  __syncthreads();
  gate_products<S::PQ>(sm.g, sm.M, sm.gam, sm.gm1, sm.m31, tid);
  {
    // P = M o (Q K^T): wave w, block (w >> 1, w & 1) (the upper one is zero)
    const int t0 = 16 * (w >> 1), s0 = 16 * (w & 1);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    if (t0 >= s0)
      acc = mm16<D>([&](int r, int k) { return sm.Qm[t0 + r][k]; }, [&](int k, int c) { return sm.K[s0 + c][k]; },
                    lane, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int t = t0 + 4 * (lane >> 4) + r, s = s0 + (lane & 15);
      sm.P[t][s] = sm.M[t][s] * acc[r];
    }
  }
  for (int jb = 0; jb < NJB; ++jb) {
    Vs.store(sm.V, tid);
    Hs.store(sm.hin, tid);
    __syncthreads();   // (also: P, for the first block)
    if (jb + 1 < NJB) {
      Vs.load(p.v + off + (jb + 1) * kJB, stride, tid);
      load_entering_rows<D, NT>(Hs, p, cp, (jb + 1) * kJB, tid);
    }
    // Y[t][j] = sum_{s <= t} P[t][s] V[s][j] + gam_t sum_i Q[t][i] hin[j][i]:
    // wave w, block (t0, j0) = (16 (w >> 1), 16 (w & 1)) of the block's rows
    {
      const int t0 = 16 * (w >> 1), j0 = 16 * (w & 1);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      const auto fp = [&](int r, int k) { return sm.P[t0 + r][k]; };
      const auto fv = [&](int k, int c) { return sm.V[k][j0 + c]; };
      acc = t0 == 0 ? mm16r<0, 16>(fp, fv, lane, acc) : mm16r<0, Q>(fp, fv, lane, acc);
      acc = mm16<D>([&](int r, int k) { return sm.gam[t0 + r] * sm.Qm[t0 + r][k]; },
                    [&](int k, int c) { return sm.hin[j0 + c][k]; }, lane, acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + 4 * (lane >> 4) + r;
        p.y[((cp.row0 + t) * p.H + cp.h) * D + jb * kJB + j0 + (lane & 15)] = acc[r];
      }
    }
    __syncthreads();   // the next block's stores overwrite V and hin
  }
}

template <int D>
struct alignas(16) GlaGradStreamSmem {
  static constexpr int PD = D + 4, PQ = Q + 4, PB = kJB + 4, NIB = D / 16;
  float Qm[Q][PD], K[Q][PD];
  float M[Q][PQ], CB[Q][PQ], G2[Q][PQ];
  float GH[Q][PD], UL[Q][PD];
  float V[Q][PB], G[Q][PB];              // v, dY of the block [t][j]
  float hin[kJB][PD], lam[kJB][PD];      // the entering state's and the adjoint's rows of the block [j][i]
  float g[Q], gam[Q], gm1[Q], m31[Q];
  float Xp[NIB][Q], Yp[NIB][Q];          // per column-block row sums of GH o Q and UL o K
  float HpP[2][Q];
  float trw[kGlaStreamGradWaves];
};

template <typename InT, int D>
__global__ __launch_bounds__(kGlaStreamGradThreads) void gla_grad_stream_kernel(GlaArgsT<InT> p) {
  constexpr int NT = kGlaStreamGradThreads, NW = kGlaStreamGradWaves, NJB = D / kJB, NIB = D / 16;
  constexpr int NACC = 4 + 4 * NIB;   // accumulated blocks: G2 (4), GH (2 NIB), UL (2 NIB)
  constexpr int MPW = (NACC + NW - 1) / NW;
  using S = GlaGradStreamSmem<D>;
  __shared__ S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l15 = lane & 15, l4 = lane >> 4;
  const ChunkPos cp = chunk_pos(p.H, p.L, p.nC);
  const int64_t off = (cp.row0 * p.H + cp.h) * D, stride = (int64_t)p.H * D;
  const int64_t soff = (cp.bh * p.nC + cp.c) * D * D;   // this chunk's adjoint slot
  Slab<Q, kJB, NT> Vs, Gs;
  Slab<kJB, D, NT> Hs, Ls;
  {
    Slab<Q, D, NT> Qs, Ks;
    Qs.load(p.q + off, stride, tid);
    Ks.load(p.k + off, stride, tid);
    Vs.load(p.v + off, stride, tid);
    Gs.load(p.dy + off, stride, tid);
    load_entering_rows<D, NT>(Hs, p, cp, 0, tid);
    Ls.load(p.lamws + soff, D, tid);
    const float gv = rr::ld(p.g, (cp.row0 + (tid & (Q - 1))) * p.H + cp.h);
    Qs.store(sm.Qm, tid);
    Ks.store(sm.K, tid);
    if (tid < Q) sm.g[tid] = gv;
  }
  __syncthreads();
  gate_products<S::PQ>(sm.g, sm.M, sm.gam, sm.gm1, sm.m31, tid);
  if (w < 4) {   // CB = Q K^T (lower blocks; the upper one is masked everywhere it is used)
    const int t0 = 16 * (w >> 1), s0 = 16 * (w & 1);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    if (t0 >= s0)
      acc = mm16<D>([&](int r, int k) { return sm.Qm[t0 + r][k]; }, [&](int k, int c) { return sm.K[s0 + c][k]; },
                    lane, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.CB[t0 + 4 * l4 + r][s0 + l15] = acc[r];
  }
  // accumulated blocks of this wave: b = w + NW m (b < NACC); dv blocks of a
  // j-block (2 row blocks s x 2 column blocks j): waves NW - 4 .. NW - 1
  f32x4_t acc[MPW];
#pragma unroll
  for (int m = 0; m < MPW; ++m) acc[m] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float trs = 0.f;
  for (int jb = 0; jb < NJB; ++jb) {
    Vs.store(sm.V, tid);
    Gs.store(sm.G, tid);
    Hs.store(sm.hin, tid);
    Ls.store(sm.lam, tid);
    __syncthreads();   // (also: CB, for the first block)
    if (jb + 1 < NJB) {
      Vs.load(p.v + off + (jb + 1) * kJB, stride, tid);
      Gs.load(p.dy + off + (jb + 1) * kJB, stride, tid);
      load_entering_rows<D, NT>(Hs, p, cp, (jb + 1) * kJB, tid);
      Ls.load(p.lamws + soff + (int64_t)(jb + 1) * kJB * D, D, tid);
    }
#pragma unroll
    for (int m = 0; m < MPW; ++m) {
      const int b = w + NW * m;
      if (b >= NACC) continue;
      if (b < 4) {   // G2[t][s] += sum_j dY[t][j] V[s][j]
        const int t0 = 16 * (b >> 1), s0 = 16 * (b & 1);
        if (t0 >= s0)
          acc[m] = mm16<kJB>([&](int r, int k) { return sm.G[t0 + r][k]; },
                             [&](int k, int c) { return sm.V[s0 + c][k]; }, lane, acc[m]);
      } else {
        const int kind = (b - 4) / (2 * NIB), rem = (b - 4) % (2 * NIB);
        const int t0 = 16 * (rem / NIB), i0 = 16 * (rem % NIB);
        if (kind == 0)   // GH[t][i] += sum_j dY[t][j] h_in[j][i]
          acc[m] = mm16<kJB>([&](int r, int k) { return sm.G[t0 + r][k]; },
                             [&](int k, int c) { return sm.hin[k][i0 + c]; }, lane, acc[m]);
        else             // UL[s][i] += sum_j V[s][j] lam[j][i]
          acc[m] = mm16<kJB>([&](int r, int k) { return sm.V[t0 + r][k]; },
                             [&](int k, int c) { return sm.lam[k][i0 + c]; }, lane, acc[m]);
      }
    }
    if (w >= NW - 4) {
      // dv[s][j] = sum_{t >= s} M[t][s] CB[t][s] dY[t][j] + m31_s sum_i K[s][i] lam[j][i]
      const int v = w - (NW - 4), s0 = 16 * (v >> 1), j0 = 16 * (v & 1);
      f32x4_t dv = {0.f, 0.f, 0.f, 0.f};
      const auto fa = [&](int r, int k) { return sm.M[k][s0 + r] * sm.CB[k][s0 + r]; };
      const auto fb = [&](int k, int c) { return sm.G[k][j0 + c]; };
      dv = s0 == 0 ? mm16r<0, Q>(fa, fb, lane, dv) : mm16r<16, Q>(fa, fb, lane, dv);
      f32x4_t kl = {0.f, 0.f, 0.f, 0.f};
      kl = mm16<D>([&](int r, int k) { return sm.K[s0 + r][k]; }, [&](int k, int c) { return sm.lam[j0 + c][k]; },
                   lane, kl);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = s0 + 4 * l4 + r;
        rr::st(p.dv, ((cp.row0 + s) * p.H + cp.h) * D + jb * kJB + j0 + l15, dv[r] + sm.m31[s] * kl[r]);
      }
    }
#pragma unroll
    for (int j = 0; j < (kJB * D + NT - 1) / NT; ++j) {   // tr = sum lam o h_in
      const int i = tid + NT * j;
      if (kJB * D % NT == 0 || i < kJB * D) trs += sm.lam[i / D][i % D] * sm.hin[i / D][i % D];
    }
    __syncthreads();   // the next block's stores overwrite the staging
  }
  // the accumulated blocks into LDS, with the X / Y row-sum partials
#pragma unroll
  for (int m = 0; m < MPW; ++m) {
    const int b = w + NW * m;
    if (b >= NACC) continue;
    if (b < 4) {
      const int t0 = 16 * (b >> 1), s0 = 16 * (b & 1);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.G2[t0 + 4 * l4 + r][s0 + l15] = acc[m][r];
    } else {
      const int kind = (b - 4) / (2 * NIB), rem = (b - 4) % (2 * NIB);
      const int t0 = 16 * (rem / NIB), ib = rem % NIB, i0 = 16 * ib;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + 4 * l4 + r;
        if (kind == 0) {
          sm.GH[t][i0 + l15] = acc[m][r];
          const float x = rr::row16_sum(acc[m][r] * sm.Qm[t][i0 + l15]);
          if (l15 == 0) sm.Xp[ib][t] = x;
        } else {
          sm.UL[t][i0 + l15] = acc[m][r];
          const float y = rr::row16_sum(acc[m][r] * sm.K[t][i0 + l15]);
          if (l15 == 0) sm.Yp[ib][t] = y;
        }
      }
    }
  }
  {
    const float t = rr::wave_sum(trs);
    if (lane == 0) sm.trw[w] = t;
  }
  __syncthreads();
  // dq[t][i] = gam_t GH[t][i] + sum_{s <= t} M[t][s] G2[t][s] K[s][i];
  // dk[s][i] = sum_{t >= s} M[t][s] G2[t][s] Q[t][i] + m31_s UL[s][i];
  // then the dg column sums of W2 = E Mh (E = CB o G2): blocks 0 .. 4 NIB + 2
  for (int blk = w; blk < 4 * NIB + 3; blk += NW) {
    if (blk < 4 * NIB) {
      const int kind = blk / (2 * NIB), rem = blk % (2 * NIB);
      const int r0 = 16 * (rem / NIB), i0 = 16 * (rem % NIB);
      f32x4_t a4 = {0.f, 0.f, 0.f, 0.f};
      if (kind == 0) {
        const auto fa = [&](int r, int k) { return sm.M[r0 + r][k] * sm.G2[r0 + r][k]; };
        const auto fb = [&](int k, int c) { return sm.K[k][i0 + c]; };
        a4 = r0 == 0 ? mm16r<0, 16>(fa, fb, lane, a4) : mm16r<0, Q>(fa, fb, lane, a4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = r0 + 4 * l4 + r;
          rr::st(p.dq, ((cp.row0 + t) * p.H + cp.h) * D + i0 + l15, a4[r] + sm.gam[t] * sm.GH[t][i0 + l15]);
        }
      } else {
        const auto fa = [&](int r, int k) { return sm.M[k][r0 + r] * sm.G2[k][r0 + r]; };
        const auto fb = [&](int k, int c) { return sm.Qm[k][i0 + c]; };
        a4 = r0 == 0 ? mm16r<0, Q>(fa, fb, lane, a4) : mm16r<16, Q>(fa, fb, lane, a4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int s = r0 + 4 * l4 + r;
          rr::st(p.dk, ((cp.row0 + s) * p.H + cp.h) * D + i0 + l15, a4[r] + sm.m31[s] * sm.UL[s][i0 + l15]);
        }
      }
    } else {
      // W2[t'][t] = sum_{s < t} E[t'][s] M[t-1][s]; column sums over t' of
      // M[t'][t] (W2 + X[t'] gam_{t-1}) for rows tp0 .. tp0 + 15
      const int v = blk - 4 * NIB, tp0 = v == 0 ? 0 : 16, t0 = v == 2 ? 16 : 0;
      f32x4_t a4 = {0.f, 0.f, 0.f, 0.f};
      const auto fa = [&](int r, int k) { return sm.CB[tp0 + r][k] * sm.G2[tp0 + r][k]; };
      const auto fb = [&](int k, int c) {
        const int t = t0 + c;
        return k < t ? sm.M[t - 1][k] : 0.f;
      };
      a4 = t0 == 0 ? mm16r<0, 16>(fa, fb, lane, a4) : mm16r<0, Q>(fa, fb, lane, a4);
      const int t = t0 + l15;
      float cs = 0.f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int tp = tp0 + 4 * l4 + r;
        float x = 0.f;
#pragma unroll
        for (int ib = 0; ib < NIB; ++ib) x += sm.Xp[ib][tp];
        cs += sm.M[tp][t] * (a4[r] + x * sm.gm1[t]);
      }
      cs += __shfl_xor(cs, 16);
      cs += __shfl_xor(cs, 32);
      if (l4 == 0) sm.HpP[tp0 / 16][t] = cs;
    }
  }
  __syncthreads();
  // dg_t = the column sums + m31_t (P_t + gam_{t-1} tr), P_t = sum_{s < t} M[t-1][s] Y_s
  if (tid < Q) {
    const int t = tid;
    float tr = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) tr += sm.trw[ww];
    float pt = 0.f;
    for (int s = 0; s < t; ++s) {
      float y = 0.f;
#pragma unroll
      for (int ib = 0; ib < NIB; ++ib) y += sm.Yp[ib][s];
      pt += sm.M[t - 1][s] * y;
    }
    const float hp = (t < 16 ? sm.HpP[0][t] : 0.f) + sm.HpP[1][t];
    rr::st(p.dg, (cp.row0 + t) * p.H + cp.h, hp + sm.m31[t] * (pt + sm.gm1[t] * tr));
  }
}

template <typename InT, int D>
int launch(const rr::GlaDenseArgs& a, int what, hipStream_t s) {
  GlaArgsT<InT> p;
  p.q = static_cast<const InT*>(a.q);
  p.k = static_cast<const InT*>(a.k);
  p.v = static_cast<const InT*>(a.v);
  p.g = static_cast<const InT*>(a.g);
  p.h0 = a.h0;
  p.ckpt = a.ckpt;
  p.lamws = a.lamws;
  p.dy = a.dy;
  p.y = a.y;
  p.dq = static_cast<InT*>(a.dq);
  p.dk = static_cast<InT*>(a.dk);
  p.dv = static_cast<InT*>(a.dv);
  p.dg = static_cast<InT*>(a.dg);
  p.mapE = a.mapE;
  p.mapP = a.mapP;
  p.B = a.B; p.L = a.L; p.H = a.H; p.nC = a.nC;
  const dim3 grid((unsigned)((int64_t)a.B * a.H * a.nC));
  switch (what) {
    case rr::kDenseMapsFwd:
      hipLaunchKernelGGL((gla_map_kernel<InT, D, false>), grid, dim3(kGlaSmallThreads), 0, s, p);
      break;
    case rr::kDenseMapsBwd:
      hipLaunchKernelGGL((gla_map_kernel<InT, D, true>), grid, dim3(kGlaSmallThreads), 0, s, p);
      break;
    case rr::kDenseOut:
      if constexpr (D > 64)
        hipLaunchKernelGGL((gla_out_stream_kernel<InT, D>), grid, dim3(kGlaStreamOutThreads), 0, s, p);
      else
        hipLaunchKernelGGL((gla_out_kernel<InT, D>), grid, dim3(kGlaSmallThreads), 0, s, p);
      break;
    default:
      if constexpr (D > 64)
        hipLaunchKernelGGL((gla_grad_stream_kernel<InT, D>), grid, dim3(kGlaStreamGradThreads), 0, s, p);
      else
        hipLaunchKernelGGL((gla_grad_kernel<InT, D>), grid, dim3(kGlaGradThreads), 0, s, p);
      break;
  }
  return rr::check_launch(what == rr::kDenseOut    ? "gla dense forward"
                          : what == rr::kDenseGrad ? "gla dense backward"
                                                   : "gla dense chunk maps");
}

template <typename InT>
int launch_shape(const rr::GlaDenseArgs& a, int what, hipStream_t s) {
  switch (a.D) {
    case 32: return launch<InT, 32>(a, what, s);
    case 64: return launch<InT, 64>(a, what, s);
    case 128: return launch<InT, 128>(a, what, s);
    default: return rr::fail(RR_EUNSUPPORTED, "gla dense: unsupported Dh");
  }
}

}  // namespace

namespace rr {

bool gla_dense_supported(int64_t T, int64_t Dh, int64_t B, int64_t H, int64_t nC) {
  return T == Q && (Dh == 32 || Dh == 64 || Dh == 128) && B * H * nC < ((int64_t)1 << 31);
}

int gla_dense_launch(const GlaDenseArgs& a, int dtype, int what, hipStream_t s) {
  switch (dtype) {
    case RR_F32: return launch_shape<float>(a, what, s);
    case RR_BF16: return launch_shape<bf16>(a, what, s);
    case RR_F16: return launch_shape<f16>(a, what, s);
    default: return fail(RR_EINVAL, "gla dense: unsupported dtype");
  }
}

}  // namespace rr
