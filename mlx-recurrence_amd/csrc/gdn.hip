// gdn.hip — Gated DeltaNet scan on gfx950 (the reference's designed next
// plug-in, docs/DESIGN_gated_deltanet.md; not code in the reference).
//
// Per (batch, head) the state is S [Dh(i)][Dh(j)] (reference :56-90):
//   p_t = k_t^T S_{t-1}                                   (per column j)
//   S_t = alpha_t (S_{t-1} - beta_t k_t p_t^T) + beta_t k_t v_t^T
//   o_t = S_t^T q_t                                       (o_t[j] = sum_i q_t[i] S_t[i][j])
// and its adjoint, newest to oldest (reference :334-440), dS = dL/dS_t:
//   dS += q_t go_t^T;  dq_t = S_t go_t;  d = k_t^T dS;  dv_t = beta d;
//   dk_t = dS (beta v - alpha beta p) - alpha beta S_{t-1} d;
//   dbeta_t = d . (v - alpha p);  dalpha_t = <dS, S_{t-1}> - beta d . p;
//   dS <- alpha (dS - beta k_t d^T).
//
// The transition alpha (I - beta k k^T) is a full Dh x Dh matrix, so chunks do
// not compose by scalar decays: this file is the sequential form (the
// reference's own first landing, its "Phase 2"), used for fp32 / fp16 inputs,
// Dh 32 and intervals of 8 or 16; bf16 inputs at Dh 64 and T 32 run the
// chunkwise (WY) form of gdn_chunk.hip instead.  The sequential form's
// parallelism is across state columns and, given checkpoints, across time
// intervals:
//   * every column j of S evolves on its own (p_j, S[:, j] and y[j] need only
//     column j), and so does every column of the adjoint (the dS recursion
//     involves neither S nor p);
//   * only the gradients couple the columns (dq, dk are row sums over j;
//     dalpha, dbeta sums over j).
// Hence three kernels:
//   1. forward: one single-wave workgroup per (head, CPW columns); a column's
//      64 / CPW adjacent lanes hold R rows each, so a column dot over i is R
//      in-lane products plus a sum over those lanes (DPP steps within a
//      16-lane row, no LDS); the step inputs are staged through the wave's
//      LDS 32 steps at a time, a block ahead; the state is checkpointed every
//      T steps;
//   2. the adjoint pass, with the same decomposition, walks the steps
//      backwards from dL/dS_{L-1} and writes the adjoint entering every
//      interval from its right (workspace [B,H,nC,Dh,Dh]) and dh0;
//   3. the gradient pass: one workgroup of Dh/8 waves per (head, interval),
//      every interval at once; it recomputes the interval's states from the
//      forward checkpoint in two levels (the state entering every group of 4
//      steps, then each group, last first, into registers), replays the
//      adjoint from the pass-2 value and forms every gradient; dq and dk are
//      reduced over a wave's 8 columns by a reduce-scatter and over the waves
//      through LDS, dalpha and dbeta over columns and waves likewise, in a
//      fixed order (deterministic).
#include "rr_common.h"
#include "rr_internal.h"
#include "rr_mfma.h"

#include <string>

namespace {

constexpr int kU = 4;   // steps per recompute group of the gradient pass

// Sum over the 8 lanes of a column (lanes 8 c .. 8 c + 7), returned in all of
// them with the same rounding (each step adds two equal pairs).
__device__ __forceinline__ float col_sum(float v) {
  v += rr::dpp_mov<0xB1>(v);    // quad_perm [1, 0, 3, 2]
  v += rr::dpp_mov<0x4E>(v);    // quad_perm [2, 3, 0, 1]
  v += rr::dpp_mov<0x141>(v);   // row_half_mirror: quad 0 <-> quad 1 of each 8
  return v;
}

// Sum over the 16 lanes of a column (lanes 16 c .. 16 c + 15) for the
// four-column waves of the column-split passes; same rounding in every lane.
__device__ __forceinline__ float col_sum16(float v) { return rr::row16_sum(v); }
template <int LPC>
__device__ __forceinline__ float col_sum_n(float v) {
  if constexpr (LPC == 16) return col_sum16(v);
  else return col_sum(v);
}

// R consecutive elements (a row run of q or k) into fp32.
template <typename InT, int R>
__device__ __forceinline__ void load_run(const InT* p, float (&out)[R]) {
  constexpr int BYTES = R * (int)sizeof(InT);
  constexpr int AL = BYTES >= 16 ? 16 : BYTES;
  const InT* a = static_cast<const InT*>(__builtin_assume_aligned(p, AL));
  InT tmp[R];
  __builtin_memcpy(tmp, a, BYTES);
#pragma unroll
  for (int r = 0; r < R; ++r) out[r] = rr::to_f32(tmp[r]);
}

// The inputs of one step for this lane: its R rows of k (and q), its column's
// v (or the output cotangent), and the step scalars.
template <int R>
struct StepIn {
  float k[R], q[R];
  float x;      // v[j] (forward, gradient pass) or dy[j] (adjoint pass)
  float a, b;
};
// WANT_Q: load q as well; FROM_DY: x is dy[j] (adjoint pass), else v[j].
template <typename InT, int R, bool WANT_Q, bool FROM_DY>
__device__ __forceinline__ StepIn<R> load_step(const InT* q, const InT* k, const InT* v, const float* dy,
                                               const InT* alpha, const InT* beta, int64_t row, int DH, int i0,
                                               int j) {
  StepIn<R> s;
  load_run<InT, R>(k + row * DH + i0, s.k);
  if constexpr (WANT_Q) {
    load_run<InT, R>(q + row * DH + i0, s.q);
  } else {
#pragma unroll
    for (int r = 0; r < R; ++r) s.q[r] = 0.f;
  }
  if constexpr (FROM_DY) s.x = dy[row * DH + j];
  else s.x = rr::ld(v, row * DH + j);
  s.a = rr::ld(alpha, row);
  s.b = rr::ld(beta, row);
  return s;
}

// sum_r x[r] y[r] as a balanced tree (depth log2 R, not R).
template <int R>
__device__ __forceinline__ float dot(const float (&x)[R], const float (&y)[R]) {
  float t[R];
#pragma unroll
  for (int r = 0; r < R; ++r) t[r] = x[r] * y[r];
#pragma unroll
  for (int w = 1; w < R; w *= 2)
#pragma unroll
    for (int r = 0; r + w < R; r += 2 * w) t[r] += t[r + w];
  return t[0];
}

// One step of the recurrence on this lane's R entries of column j; returns p.
template <int R, int LPC = 8>
__device__ __forceinline__ float step(float (&S)[R], const StepIn<R>& in) {
  const float p = col_sum_n<LPC>(dot<R>(in.k, S));       // p_j = k^T S_{t-1} (reference :75-84)
  // S <- alpha (S - beta k p) + beta k v = alpha S + k (beta v - alpha beta p)
  const float cc = in.b * in.x - in.a * (in.b * p);
#pragma unroll
  for (int r = 0; r < R; ++r) S[r] = in.a * S[r] + in.k[r] * cc;
  return p;
}

// One step of the adjoint recursion on this lane's R entries of column j
// (dS += q go^T; d = k^T dS; dS <- alpha (dS - beta k d^T)); returns d.
template <int R, int LPC = 8>
__device__ __forceinline__ float adjoint_step(float (&adj)[R], const float (&q)[R], const float (&k)[R], float go,
                                              float a, float b) {
#pragma unroll
  for (int r = 0; r < R; ++r) adj[r] += q[r] * go;
  const float d = col_sum_n<LPC>(dot<R>(k, adj));
  const float abd = a * (b * d);
#pragma unroll
  for (int r = 0; r < R; ++r) adj[r] = a * adj[r] - k[r] * abd;   // alpha (dS - beta k d^T)
  return d;
}

// The forward and adjoint passes run one single-wave workgroup per (head,
// CPW-column block): B H Dh/CPW waves spread over the GPU.  A step is a chain
// of dependent instructions per lane, so the split that gives each lane the
// fewest (R = Dh CPW / 64 rows of one column, the column's 64 / CPW lanes
// adjacent, CPW = 4 for Dh = 64) runs fastest.  The wave's step inputs are
// staged through LDS kTS steps at a time, double-buffered: the next block's
// loads are issued into registers a whole block ahead and written to LDS at
// the block's end.  The column blocks of one head share an XCD (their inputs
// stay in one L2).
constexpr int kTS = 32;

template <int DH, int CPW>
struct StageSmem {
  float k[2][kTS][DH], q[2][kTS][DH];
  float x[2][kTS][CPW];   // v or dy of this wave's columns
  float a[2][kTS], b[2][kTS];
};

struct ColId {
  int bh, jb;
  bool valid;
};
__device__ __forceinline__ ColId col_id(int NJ, int BH) {
  const int id = blockIdx.x, xcd = id % 8, k = id / 8;
  const int bh = (k / NJ) * 8 + xcd;
  return ColId{bh, k % NJ, bh < BH};
}
inline unsigned col_grid(int64_t BH, int NJ) { return (unsigned)((BH + 7) / 8 * 8 * NJ); }

// A raw run of N elements (N = 4 or 8: 8 to 32 bytes), then widened into LDS.
template <typename E, int N>
__device__ __forceinline__ void ldn(const E* p, uint4 (&r)[2]) {
  constexpr int BYTES = N * (int)sizeof(E), AL = BYTES >= 16 ? 16 : BYTES;
  __builtin_memcpy(r, __builtin_assume_aligned(p, AL), BYTES);
}
template <typename E, int N>
__device__ __forceinline__ void stn(float* dst, const uint4 (&r)[2]) {
  E tmp[N];
  __builtin_memcpy(tmp, r, N * sizeof(E));
#pragma unroll
  for (int e = 0; e < N; e += 4)
    reinterpret_cast<float4*>(dst)[e / 4] =
        make_float4(rr::to_f32(tmp[e]), rr::to_f32(tmp[e + 1]), rr::to_f32(tmp[e + 2]), rr::to_f32(tmp[e + 3]));
}

// One block's loads held by the wave's lanes: the k and q rows (kTS DH / 8
// runs of 8 each), the wave's CPW columns of x per step (kTS runs) and the
// step scalars.
template <typename InT, typename XT, int DH, int CPW>
struct Stager {
  static constexpr int CPA = kTS * DH / 8;                 // runs per k / q block
  static constexpr int NCH = 2 * CPA + kTS;
  static constexpr int PER = (NCH + 63) / 64;
  uint4 raw[PER][2];
  float sc;
  __device__ __forceinline__ void issue(const InT* q, const InT* k, const XT* x, const InT* alpha, const InT* beta,
                                        int blk, int64_t row0, int H, int L, int j0, int lane) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int id = lane + 64 * i;
      if (id < 2 * CPA) {
        const int rem = id % CPA, st = rem / (DH / 8), ch = rem % (DH / 8), t = blk * kTS + st;
        if (t < L) ldn<InT, 8>((id < CPA ? k : q) + (row0 + (int64_t)t * H) * DH + 8 * ch, raw[i]);
      } else if (id < NCH) {
        const int st = id - 2 * CPA, t = blk * kTS + st;
        if (t < L) ldn<XT, CPW>(x + (row0 + (int64_t)t * H) * DH + j0, raw[i]);
      }
    }
    sc = 0.f;
    const int t = blk * kTS + (lane % kTS);
    if (t < L) sc = rr::ld(lane < kTS ? alpha : beta, row0 + (int64_t)t * H);
  }
  __device__ __forceinline__ void commit(StageSmem<DH, CPW>& sm, int buf, int blk, int L, int lane) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int id = lane + 64 * i;
      if (id < 2 * CPA) {
        const int rem = id % CPA, st = rem / (DH / 8), ch = rem % (DH / 8);
        if (blk * kTS + st < L) stn<InT, 8>(id < CPA ? &sm.k[buf][st][8 * ch] : &sm.q[buf][st][8 * ch], raw[i]);
      } else if (id < NCH) {
        const int st = id - 2 * CPA;
        if (blk * kTS + st < L) stn<XT, CPW>(&sm.x[buf][st][0], raw[i]);
      }
    }
    (lane < kTS ? sm.a : sm.b)[buf][lane % kTS] = sc;
  }
};

template <int R, int DH, int CPW>
__device__ __forceinline__ StepIn<R> stage_step(const StageSmem<DH, CPW>& sm, int buf, int st, int i0, int c) {
  StepIn<R> in;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    in.k[r] = sm.k[buf][st][i0 + r];
    in.q[r] = sm.q[buf][st][i0 + r];
  }
  in.x = sm.x[buf][st][c];
  in.a = sm.a[buf][st];
  in.b = sm.b[buf][st];
  return in;
}

template <int DH>
constexpr int kCpw = DH == 64 ? 4 : 8;   // columns per wave of the column-split passes

template <typename InT, int DH>
__global__ __launch_bounds__(64) void gdn_fwd_kernel(const InT* __restrict__ q, const InT* __restrict__ k,
                                                     const InT* __restrict__ v, const InT* __restrict__ alpha,
                                                     const InT* __restrict__ beta, const float* __restrict__ h0,
                                                     float* __restrict__ y, float* __restrict__ ckpt, int BH, int H,
                                                     int L, int T, int nC) {
  constexpr int CPW = kCpw<DH>, LPC = 64 / CPW, R = DH / LPC, NJ = DH / CPW;
  __shared__ StageSmem<DH, CPW> sm;
  const ColId id = col_id(NJ, BH);
  if (!id.valid) return;
  const int bh = id.bh, b = bh / H, h = bh % H;
  const int lane = threadIdx.x, g = lane % LPC, c = lane / LPC, j = CPW * id.jb + c, i0 = R * g;
  const int64_t row0 = (int64_t)b * L * H + h;   // (b, t = 0, h); step t adds t H
  const int logT = __builtin_ctz(T);
  Stager<InT, InT, DH, CPW> stg;
  float S[R];
#pragma unroll
  for (int r = 0; r < R; ++r) S[r] = h0 != nullptr ? h0[((int64_t)bh * DH + i0 + r) * DH + j] : 0.f;
  const int nblk = (L + kTS - 1) / kTS;
  stg.issue(q, k, v, alpha, beta, 0, row0, H, L, CPW * id.jb, lane);
  stg.commit(sm, 0, 0, L, lane);
  if (nblk > 1) stg.issue(q, k, v, alpha, beta, 1, row0, H, L, CPW * id.jb, lane);
  rr::wave_lds_sync();
  for (int blk = 0; blk < nblk; ++blk) {
    const int buf = blk & 1, tn = min(kTS, L - blk * kTS);
    // four steps per pass (tn is a multiple of 8): their LDS reads all go out first
    for (int st0 = 0; st0 < tn; st0 += 4) {
      StepIn<R> in[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) in[u] = stage_step<R, DH, CPW>(sm, buf, st0 + u, i0, c);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = blk * kTS + st0 + u;
        step<R, LPC>(S, in[u]);
        const float o = col_sum_n<LPC>(dot<R>(in[u].q, S));   // o_t[j] = sum_i q_t[i] S_t[i][j] (:86-90)
        if (g == 0) y[(row0 + (int64_t)t * H) * DH + j] = o;
        if (((t + 1) & (T - 1)) == 0) {                  // T is a power of two
          float* ck = ckpt + (((int64_t)bh * nC + ((t + 1) >> logT) - 1) * DH + i0) * DH + j;
#pragma unroll
          for (int r = 0; r < R; ++r) ck[r * DH] = S[r];
        }
      }
    }
    if (blk + 1 < nblk) {
      stg.commit(sm, buf ^ 1, blk + 1, L, lane);
      if (blk + 2 < nblk) stg.issue(q, k, v, alpha, beta, blk + 2, row0, H, L, CPW * id.jb, lane);
    }
    rr::wave_lds_sync();
  }
}

// Adjoint pass: adjck[bh, c] = dL/dS at the end of interval c from the later
// steps only (what the gradient pass of interval c starts from); dh0.  The
// blocks are staged and walked last first.
template <typename InT, int DH>
__global__ __launch_bounds__(64) void gdn_adj_kernel(const float* __restrict__ dy, const float* __restrict__ dfinal,
                                                     const InT* __restrict__ q, const InT* __restrict__ k,
                                                     const InT* __restrict__ alpha, const InT* __restrict__ beta,
                                                     float* __restrict__ adjck, float* __restrict__ dh0, int BH,
                                                     int H, int L, int T, int nC) {
  constexpr int CPW = kCpw<DH>, LPC = 64 / CPW, R = DH / LPC, NJ = DH / CPW;
  __shared__ StageSmem<DH, CPW> sm;
  const ColId id = col_id(NJ, BH);
  if (!id.valid) return;
  const int bh = id.bh, b = bh / H, h = bh % H;
  const int lane = threadIdx.x, g = lane % LPC, c = lane / LPC, j = CPW * id.jb + c, i0 = R * g;
  const int64_t row0 = (int64_t)b * L * H + h;
  const int logT = __builtin_ctz(T);
  Stager<InT, float, DH, CPW> stg;
  float adj[R];
#pragma unroll
  for (int r = 0; r < R; ++r) adj[r] = dfinal != nullptr ? dfinal[((int64_t)bh * DH + i0 + r) * DH + j] : 0.f;
  const int nblk = (L + kTS - 1) / kTS;
  stg.issue(q, k, dy, alpha, beta, nblk - 1, row0, H, L, CPW * id.jb, lane);
  stg.commit(sm, 0, nblk - 1, L, lane);
  if (nblk > 1) stg.issue(q, k, dy, alpha, beta, nblk - 2, row0, H, L, CPW * id.jb, lane);
  rr::wave_lds_sync();
  for (int n = 0; n < nblk; ++n) {
    const int blk = nblk - 1 - n, buf = n & 1, tn = min(kTS, L - blk * kTS);
    for (int st0 = tn - 1; st0 >= 0; st0 -= 4) {   // four steps per pass, reads first
      StepIn<R> in[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) in[u] = stage_step<R, DH, CPW>(sm, buf, st0 - u, i0, c);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int t = blk * kTS + st0 - u;
        if (((t + 1) & (T - 1)) == 0) {   // the end of interval (t + 1) / T - 1, before its own steps
          float* ac = adjck + (((int64_t)bh * nC + ((t + 1) >> logT) - 1) * DH + i0) * DH + j;
#pragma unroll
          for (int r = 0; r < R; ++r) ac[r * DH] = adj[r];
        }
        adjoint_step<R, LPC>(adj, in[u].q, in[u].k, in[u].x, in[u].a, in[u].b);
      }
    }
    if (n + 1 < nblk) {
      stg.commit(sm, buf ^ 1, blk - 1, L, lane);
      if (n + 2 < nblk) stg.issue(q, k, dy, alpha, beta, blk - 2, row0, H, L, CPW * id.jb, lane);
    }
    rr::wave_lds_sync();
  }
  if (dh0 != nullptr) {
#pragma unroll
    for (int r = 0; r < R; ++r) dh0[((int64_t)bh * DH + i0 + r) * DH + j] = adj[r];
  }
}

// Reduce-scatter over the 8 columns of a wave (lane bits 3..5, xor 32, 16, 8):
// on entry every lane holds R values (rows i0 .. i0 + R - 1 of its column); on
// return it holds the sum over the wave's columns of row i0 + `row` (rounds
// keep the half chosen by column bits 2, 1, 0; with R = 4 the last round is a
// plain pairwise sum, so two lanes hold each row).
template <int R>
__device__ __forceinline__ float col_reduce_scatter(float (&x)[R], int lane, int& row) {
  const int c = lane >> 3;
  float x2[R / 2];
  {
    const bool hi = (c & 4) != 0;
#pragma unroll
    for (int r = 0; r < R / 2; ++r) {
      const float send = hi ? x[r] : x[R / 2 + r];
      const float keep = hi ? x[R / 2 + r] : x[r];
      x2[r] = keep + __shfl_xor(send, 32, 64);
    }
  }
  int idx = (c & 4) ? R / 2 : 0;
  if constexpr (R == 8) {
    float x4[2];
    const bool hi2 = (c & 2) != 0;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float send = hi2 ? x2[r] : x2[2 + r];
      const float keep = hi2 ? x2[2 + r] : x2[r];
      x4[r] = keep + __shfl_xor(send, 16, 64);
    }
    idx += (c & 2) ? 2 : 0;
    const bool hi1 = (c & 1) != 0;
    const float send = hi1 ? x4[0] : x4[1];
    const float keep = hi1 ? x4[1] : x4[0];
    idx += (c & 1) ? 1 : 0;
    row = idx;
    return keep + __shfl_xor(send, 8, 64);
  } else {   // R == 4
    const bool hi2 = (c & 2) != 0;
    const float send = hi2 ? x2[0] : x2[1];
    const float keep = hi2 ? x2[1] : x2[0];
    idx += (c & 2) ? 1 : 0;
    row = idx;
    const float s = keep + __shfl_xor(send, 16, 64);
    return s + __shfl_xor(s, 8, 64);
  }
}

// Sum over the 8 columns of a wave, in every lane (lane bits 3..5).
__device__ __forceinline__ float wave_col_sum(float v) {
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 16, 64);
  return v + __shfl_xor(v, 32, 64);
}

template <int DH, int T>
struct GradSmem {
  float gq[T][DH / 8][DH];   // per step, per wave: dq partial sums over the wave's columns
  float gk[T][DH / 8][DH];
  float ga[T][DH / 8];       // per step, per wave: dalpha, dbeta terms of its columns
  float gb[T][DH / 8];
};

// Gradient pass: one workgroup per (head, interval); wave w owns columns
// 8 w .. 8 w + 7 with the lane layout of the column-split kernels.
template <typename InT, int DH, int T>
__global__ __launch_bounds__(64 * (DH / 8)) void gdn_grad_kernel(
    const float* __restrict__ dy, const InT* __restrict__ q, const InT* __restrict__ k, const InT* __restrict__ v,
    const InT* __restrict__ alpha, const InT* __restrict__ beta, const float* __restrict__ h0,
    const float* __restrict__ ckpt, const float* __restrict__ adjck, InT* __restrict__ dq, InT* __restrict__ dk,
    InT* __restrict__ dv, InT* __restrict__ dalpha, InT* __restrict__ dbeta, int H, int L, int nC) {
  constexpr int R = DH / 8, NW = DH / 8, NG = T / kU;
  __shared__ GradSmem<DH, T> sm;
  const int cc = blockIdx.x % nC, bh = blockIdx.x / nC, b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int g = lane & 7, j = 8 * w + (lane >> 3), i0 = R * g;
  const int t0 = cc * T;
  float adj[R];
#pragma unroll
  for (int r = 0; r < R; ++r) adj[r] = adjck[(((int64_t)bh * nC + cc) * DH + i0 + r) * DH + j];
  // level 1: the state entering each group of kU steps
  float Sg[NG][R];
  {
    float S[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float* src = cc > 0 ? ckpt + (((int64_t)bh * nC + cc - 1) * DH + i0 + r) * DH + j
                                : (h0 != nullptr ? h0 + ((int64_t)bh * DH + i0 + r) * DH + j : nullptr);
      S[r] = src != nullptr ? *src : 0.f;
    }
#pragma unroll
    for (int gr = 0; gr < NG; ++gr) {
#pragma unroll
      for (int r = 0; r < R; ++r) Sg[gr][r] = S[r];
      if (gr + 1 < NG) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int64_t row = ((int64_t)b * L + t0 + kU * gr + u) * H + h;
          step<R>(S, load_step<InT, R, false, false>(q, k, v, nullptr, alpha, beta, row, DH, i0, j));
        }
      }
    }
  }
  // level 2: each group recomputed into registers, then swept backwards
#pragma unroll
  for (int gr = NG - 1; gr >= 0; --gr) {
    float St[kU][R];
    StepIn<R> in[kU];
    float pv[kU];
    {
      float S[R];
#pragma unroll
      for (int r = 0; r < R; ++r) S[r] = Sg[gr][r];
#pragma unroll
      for (int u = 0; u < kU; ++u) {
        const int64_t row = ((int64_t)b * L + t0 + kU * gr + u) * H + h;
        in[u] = load_step<InT, R, true, false>(q, k, v, nullptr, alpha, beta, row, DH, i0, j);
        pv[u] = step<R>(S, in[u]);
#pragma unroll
        for (int r = 0; r < R; ++r) St[u][r] = S[r];
      }
    }
#pragma unroll
    for (int u = kU - 1; u >= 0; --u) {
      const int tl = kU * gr + u;   // step within the interval
      const int64_t row = ((int64_t)b * L + t0 + tl) * H + h;
      const float go = dy[row * DH + j];
      const float a = in[u].a, bb = in[u].b, p = pv[u];
      float gq[R], gk[R];
#pragma unroll
      for (int r = 0; r < R; ++r) gq[r] = St[u][r] * go;   // dq = S_t go
      // the adjoint step as in the adjoint pass, keeping dS (after the q go^T
      // term) for the terms below
      float adjt[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        adj[r] += in[u].q[r] * go;                         // dS += q go^T
        adjt[r] = adj[r];
      }
      const float d = col_sum(dot<R>(in[u].k, adjt));      // d_j = k^T dS
      const float ad = a * (bb * d);
#pragma unroll
      for (int r = 0; r < R; ++r) adj[r] = a * adj[r] - in[u].k[r] * ad;   // dS <- alpha (dS - beta k d^T)
      const float wk = bb * in[u].x - a * (bb * p);
      float sp[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        sp[r] = u > 0 ? St[u - 1][r] : Sg[gr][r];          // S_{t-1}
        gk[r] = adjt[r] * wk - sp[r] * ad;                 // dk terms
      }
      const float sa = col_sum(dot<R>(adjt, sp));          // <dS, S_{t-1}> over this column
      if (g == 0) rr::st(dv, row * DH + j, bb * d);        // dv = beta d
      const float ga = wave_col_sum(g == 0 ? sa - bb * d * p : 0.f);           // dalpha terms of the wave's columns
      const float gb = wave_col_sum(g == 0 ? d * (in[u].x - a * p) : 0.f);     // dbeta terms
      if (lane == 0) {
        sm.ga[tl][w] = ga;
        sm.gb[tl][w] = gb;
      }
      int rq, rk;
      const float sq = col_reduce_scatter<R>(gq, lane, rq);
      const float sk = col_reduce_scatter<R>(gk, lane, rk);
      sm.gq[tl][w][i0 + rq] = sq;
      sm.gk[tl][w][i0 + rk] = sk;
    }
  }
  __syncthreads();
  // the interval's sums over the waves, in order
  for (int e = tid; e < T * DH; e += 64 * NW) {
    const int tl = e / DH, i = e % DH;
    float sqs = 0.f, sks = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      sqs += sm.gq[tl][ww][i];
      sks += sm.gk[tl][ww][i];
    }
    const int64_t row = ((int64_t)b * L + t0 + tl) * H + h;
    rr::st(dq, row * DH + i, sqs);
    rr::st(dk, row * DH + i, sks);
  }
  for (int tl = tid; tl < T; tl += 64 * NW) {
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      sa += sm.ga[tl][ww];
      sb += sm.gb[tl][ww];
    }
    const int64_t row = ((int64_t)b * L + t0 + tl) * H + h;
    rr::st(dalpha, row, sa);
    rr::st(dbeta, row, sb);
  }
}

int check_gdn(const char* who, int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, int dtype) {
  if (B <= 0 || L <= 0 || H <= 0 || Dh <= 0) return rr::fail(RR_EINVAL, std::string(who) + ": all dimensions must be positive");
  if (int rc = rr::check_segment_shape(L, seg, Dh, "Dh")) return rc;
  if (!rr::valid_dtype(dtype)) return rr::fail(RR_EINVAL, std::string(who) + ": unsupported dtype");
  if (Dh != 32 && Dh != 64) return rr::fail(RR_EUNSUPPORTED, std::string(who) + ": Dh must be 32 or 64");
  const int64_t T = rr::chunk_len(L, seg);
  if (T != 8 && T != 16 && T != 32)
    return rr::fail(RR_EUNSUPPORTED, std::string(who) + ": seg must be a multiple of 8 (checkpoint interval 8, 16 or 32)");
  if (B * H * (L / T) >= ((int64_t)1 << 31) || B * H * Dh >= ((int64_t)1 << 30) || B * L * H * Dh >= ((int64_t)1 << 40))
    return rr::fail(RR_EUNSUPPORTED, std::string(who) + ": tensors too large");
  return RR_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

size_t adj_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg) {
  return (size_t)(B * H * (L / rr::chunk_len(L, seg)) * Dh * Dh) * sizeof(float);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// The backward's workspace: the adjoint checkpoints, then (chunkwise adjoint
// pass) every chunk's fragments.
size_t bwd_ws_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, int dtype) {
  const size_t n = adj_bytes(B, L, H, Dh, seg);
  return rr::gdn_chunk_supported(dtype, Dh, rr::chunk_len(L, seg)) ? align256(n) + rr::gdn_chunk_bwd_ws_bytes(B, L, H)
                                                                    : n;
}

template <typename InT, int DH, int T>
void launch_grad_t(const float* dy, const void* q, const void* k, const void* v, const void* alpha, const void* beta,
                   const float* h0, const float* ckpt, const float* adjck, void* dq, void* dk, void* dv, void* dalpha,
                   void* dbeta, int64_t B, int64_t H, int64_t L, int64_t nC, hipStream_t s) {
  hipLaunchKernelGGL((gdn_grad_kernel<InT, DH, T>), dim3((unsigned)(B * H * nC)), dim3(64 * (DH / 8)), 0, s, dy,
                     static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(v),
                     static_cast<const InT*>(alpha), static_cast<const InT*>(beta), h0, ckpt, adjck,
                     static_cast<InT*>(dq), static_cast<InT*>(dk), static_cast<InT*>(dv), static_cast<InT*>(dalpha),
                     static_cast<InT*>(dbeta), (int)H, (int)L, (int)nC);
}

template <typename InT, int DH>
void launch_bwd_dh(int64_t T, const float* dy, const float* dfinal, const void* q, const void* k, const void* v,
                   const void* alpha, const void* beta, const float* h0, const float* ckpt, float* adjck, void* dq,
                   void* dk, void* dv, void* dalpha, void* dbeta, float* dh0, int64_t B, int64_t H, int64_t L,
                   int64_t nC, hipStream_t s) {
  hipLaunchKernelGGL((gdn_adj_kernel<InT, DH>), dim3(col_grid(B * H, DH / kCpw<DH>)), dim3(64), 0, s, dy, dfinal,
                     static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(alpha),
                     static_cast<const InT*>(beta), adjck, dh0, (int)(B * H), (int)H, (int)L, (int)T, (int)nC);
  if (T == 32)
    launch_grad_t<InT, DH, 32>(dy, q, k, v, alpha, beta, h0, ckpt, adjck, dq, dk, dv, dalpha, dbeta, B, H, L, nC, s);
  else if (T == 16)
    launch_grad_t<InT, DH, 16>(dy, q, k, v, alpha, beta, h0, ckpt, adjck, dq, dk, dv, dalpha, dbeta, B, H, L, nC, s);
  else
    launch_grad_t<InT, DH, 8>(dy, q, k, v, alpha, beta, h0, ckpt, adjck, dq, dk, dv, dalpha, dbeta, B, H, L, nC, s);
}

}  // namespace

extern "C" size_t rr_gdn_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, int dtype) {
  if (B <= 0 || L <= 0 || H <= 0 || Dh <= 0 || rr::chunk_len(L, seg) == 0 || !rr::valid_dtype(dtype)) return 0;
  return bwd_ws_bytes(B, L, H, Dh, seg, dtype);
}

extern "C" size_t rr_gdn_fwd_workspace_bytes(int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, int dtype) {
  if (check_gdn("gdn_fwd", B, L, H, Dh, seg, dtype) != RR_OK) return 0;
  return rr::gdn_chunk_supported(dtype, Dh, rr::chunk_len(L, seg)) ? rr::gdn_chunk_ws_bytes(B, L, H) : 0;
}

extern "C" int rr_gdn_fwd(const void* q, const void* k, const void* v, const void* alpha, const void* beta, int dtype,
                          int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, const float* h0, float* y,
                          float* ckpt, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_gdn("gdn_fwd", B, L, H, Dh, seg, dtype)) return rc;
  if (!q || !k || !v || !alpha || !beta || !y || !ckpt) return rr::fail(RR_EINVAL, "gdn_fwd: null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v))
    return rr::fail(RR_EINVAL, "gdn_fwd: q, k and v must be 16-byte aligned");
  const int64_t T = rr::chunk_len(L, seg), nC = L / T;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (workspace != nullptr || workspace_bytes != 0) {   // the chunkwise form was asked for
    if (!rr::gdn_chunk_supported(dtype, Dh, T))
      return rr::fail(RR_EINVAL, "gdn_fwd: a workspace is only taken by the chunkwise form (bf16, Dh 64, T 32)");
    if (workspace == nullptr || !aligned16(workspace) || workspace_bytes < rr::gdn_chunk_ws_bytes(B, L, H))
      return rr::fail(RR_EWORKSPACE, "gdn_fwd: workspace smaller than rr_gdn_fwd_workspace_bytes or misaligned");
    return rr::gdn_chunk_fwd(q, k, v, alpha, beta, B, L, H, h0, y, ckpt, workspace, s);
  }
  RR_DISPATCH_DTYPE(dtype, {
    if (Dh == 64)
      hipLaunchKernelGGL((gdn_fwd_kernel<InT, 64>), dim3(col_grid(B * H, 64 / kCpw<64>)), dim3(64), 0, s,
                         static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(v),
                         static_cast<const InT*>(alpha), static_cast<const InT*>(beta), h0, y, ckpt, (int)(B * H),
                         (int)H, (int)L, (int)T, (int)nC);
    else
      hipLaunchKernelGGL((gdn_fwd_kernel<InT, 32>), dim3(col_grid(B * H, 32 / kCpw<32>)), dim3(64), 0, s,
                         static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(v),
                         static_cast<const InT*>(alpha), static_cast<const InT*>(beta), h0, y, ckpt, (int)(B * H),
                         (int)H, (int)L, (int)T, (int)nC);
  });
  return rr::check_launch("rr_gdn_fwd");
}

extern "C" int rr_gdn_bwd(const float* dy, const float* dfinal, const void* q, const void* k, const void* v,
                          const void* alpha, const void* beta, int dtype, int64_t B, int64_t L, int64_t H, int64_t Dh,
                          int64_t seg, const float* h0, const float* ckpt, void* dq, void* dk, void* dv,
                          void* dalpha, void* dbeta, float* dh0, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (int rc = check_gdn("gdn_bwd", B, L, H, Dh, seg, dtype)) return rc;
  if (!dy || !q || !k || !v || !alpha || !beta || !ckpt || !dq || !dk || !dv || !dalpha || !dbeta)
    return rr::fail(RR_EINVAL, "gdn_bwd: null pointer argument");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dy))
    return rr::fail(RR_EINVAL, "gdn_bwd: q, k, v and dy must be 16-byte aligned");
  if (!workspace || workspace_bytes < bwd_ws_bytes(B, L, H, Dh, seg, dtype))
    return rr::fail(RR_EWORKSPACE, "gdn_bwd: workspace too small");
  const int64_t T = rr::chunk_len(L, seg), nC = L / T;
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* adjck = static_cast<float*>(workspace);
  // bf16, Dh 64, T 32: the adjoint pass and the gradient pass in chunkwise form
  const bool chunked = rr::gdn_chunk_supported(dtype, Dh, T);
  if (chunked && !aligned16(workspace)) return rr::fail(RR_EWORKSPACE, "gdn_bwd: workspace must be 16-byte aligned");
  RR_DISPATCH_DTYPE(dtype, {
    if (chunked) {
      void* packs = static_cast<char*>(workspace) + align256(adj_bytes(B, L, H, Dh, seg));
      if (int rc = rr::gdn_chunk_adjoint(q, k, v, alpha, beta, dy, dfinal, B, L, H, adjck, dh0, packs, s)) return rc;
      if (int rc = rr::gdn_chunk_grad(dy, q, k, v, alpha, beta, h0, ckpt, adjck, dq, dk, dv, dalpha, dbeta, B, L, H, s))
        return rc;
    } else if (Dh == 64)
      launch_bwd_dh<InT, 64>(T, dy, dfinal, q, k, v, alpha, beta, h0, ckpt, adjck, dq, dk, dv, dalpha, dbeta, dh0, B,
                             H, L, nC, s);
    else
      launch_bwd_dh<InT, 32>(T, dy, dfinal, q, k, v, alpha, beta, h0, ckpt, adjck, dq, dk, dv, dalpha, dbeta, dh0, B,
                             H, L, nC, s);
  });
  return rr::check_launch("rr_gdn_bwd");
}
