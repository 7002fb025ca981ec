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
// The transition alpha (I - beta k k^T) is a full Dh x Dh matrix, so unlike
// the scalar-decay scans there is no cheap chunk composition: this is the
// sequential form (the reference's own first landing, its "Phase 2").  One
// workgroup per (batch, head) of Dh / 8 waves; wave w owns the 8 columns
// j = 8 w .. 8 w + 7, and lane l of it column j = 8 w + (l % 8) and the
// R = Dh / 8 rows i = R (l / 8) .. R (l / 8) + R - 1 of it.  The column dots
// over i (p_t, o_t, d) are in-lane sums plus a sum over the 8 lanes that hold
// one column (three cross-lane steps); the waves never wait for each other in
// the forward.  The backward's row sums over j (dq, dk) are reduced over the
// 8 columns of a wave by a reduce-scatter (each round halves the values a
// lane keeps) and over the waves through LDS once per checkpoint interval;
// dalpha, dbeta go through LDS per column.  All sums have a fixed order
// (deterministic).
//
// Checkpoints [B,H,nC,Dh(i),Dh(j)] every T steps (T = rr_chunk_len; the last
// is the final state, S[i][j] layout).  The backward recomputes each
// interval from its checkpoint in two levels: a first pass keeps the state
// entering every group of U = 4 steps, then each group (last first) is
// recomputed into registers and swept backwards: twice the forward's
// arithmetic, no state history in memory.
#include "rr_common.h"

#include <string>

namespace {

constexpr int kU = 4;   // steps per recompute group

// Sum over the lanes that share a column (lane bits 3..5: lanes l, l ^ 8, ...).
__device__ __forceinline__ float col_sum(float v) {
  v += __shfl_xor(v, 8, 64);
  v += __shfl_xor(v, 16, 64);
  v += __shfl_xor(v, 32, 64);
  return v;
}

// The inputs of one step for this lane: its R rows of k and q (q only where
// wanted), its column's v, and the scalars.
template <typename InT, int R, bool WANT_Q>
struct StepIn {
  float k[R], q[WANT_Q ? R : 1];
  float v, a, b;
};
template <typename InT, int R, bool WANT_Q>
__device__ __forceinline__ StepIn<InT, R, WANT_Q> load_step(const InT* q, const InT* k, const InT* v,
                                                            const InT* alpha, const InT* beta, int64_t row, int DH,
                                                            int i0, int j) {
  StepIn<InT, R, WANT_Q> s;
#pragma unroll
  for (int r = 0; r < R; ++r) s.k[r] = rr::ld(k, row * DH + i0 + r);
  if constexpr (WANT_Q) {
#pragma unroll
    for (int r = 0; r < R; ++r) s.q[r] = rr::ld(q, row * DH + i0 + r);
  }
  s.v = rr::ld(v, row * DH + j);
  s.a = rr::ld(alpha, row);
  s.b = rr::ld(beta, row);
  return s;
}

// One step of the recurrence on this lane's R entries of column j; returns p.
template <typename InT, int R, bool WANT_Q>
__device__ __forceinline__ float step(float (&S)[R], const StepIn<InT, R, WANT_Q>& in) {
  float p = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r) p += in.k[r] * S[r];
  p = col_sum(p);                                        // p_j = k^T S_{t-1} (reference :75-84)
  const float bv = in.b * in.v, bp = in.b * p;
#pragma unroll
  for (int r = 0; r < R; ++r) S[r] = in.a * (S[r] - in.k[r] * bp) + in.k[r] * bv;
  return p;
}

template <typename InT, int DH>
__global__ __launch_bounds__(64 * (DH / 8)) void gdn_fwd_kernel(const InT* __restrict__ q, const InT* __restrict__ k,
                                                                const InT* __restrict__ v, const InT* __restrict__ alpha,
                                                                const InT* __restrict__ beta,
                                                                const float* __restrict__ h0, float* __restrict__ y,
                                                                float* __restrict__ ckpt, int H, int L, int T, int nC) {
  constexpr int R = DH / 8;
  const int bh = blockIdx.x, b = bh / H, h = bh % H;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int j = 8 * w + (lane & 7), i0 = R * (lane >> 3);
  float S[R];
#pragma unroll
  for (int r = 0; r < R; ++r) S[r] = h0 != nullptr ? h0[((int64_t)bh * DH + i0 + r) * DH + j] : 0.f;
  // inputs run kU steps ahead of the arithmetic (a ring of kU step loads in
  // registers), so the loads' latency overlaps kU steps of cross-lane sums
  StepIn<InT, R, true> ring[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u)
    if (u < L) ring[u] = load_step<InT, R, true>(q, k, v, alpha, beta, ((int64_t)b * L + u) * H + h, DH, i0, j);
  for (int t0 = 0; t0 < L; t0 += kU) {   // L is a multiple of T, T of kU
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int t = t0 + u;
      const int64_t row = ((int64_t)b * L + t) * H + h;
      const StepIn<InT, R, true> in = ring[u];
      if (t + kU < L) ring[u] = load_step<InT, R, true>(q, k, v, alpha, beta, row + (int64_t)kU * H, DH, i0, j);
      step<InT, R, true>(S, in);
      float o = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r) o += in.q[r] * S[r];
      o = col_sum(o);                                    // o_t[j] = sum_i q_t[i] S_t[i][j] (:86-90)
      if ((lane >> 3) == 0) y[row * DH + j] = o;
      if ((t + 1) % T == 0) {
        float* ck = ckpt + (((int64_t)bh * nC + (t + 1) / T - 1) * DH + i0) * DH + j;
#pragma unroll
        for (int r = 0; r < R; ++r) ck[r * DH] = S[r];
      }
    }
  }
}

// Reduce-scatter over the 8 columns of a wave (lane bits 0..2): on entry every
// lane holds R values (rows i0 .. i0 + R - 1 of its column); on return lane
// l holds the sum over the wave's columns of row i0 + idx, idx the value
// returned in `row` (rounds keep the half chosen by column bits 2, 1, 0; with
// R = 4 the last round is a plain pairwise sum).
template <int R>
__device__ __forceinline__ float col_reduce_scatter(float (&x)[R], int lane, int& row) {
  const int c = lane & 7;
  float x2[R / 2];
  {
    const bool hi = (c & 4) != 0;
#pragma unroll
    for (int r = 0; r < R / 2; ++r) {
      const float send = hi ? x[r] : x[R / 2 + r];
      const float keep = hi ? x[R / 2 + r] : x[r];
      x2[r] = keep + __shfl_xor(send, 4, 64);
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
      x4[r] = keep + __shfl_xor(send, 2, 64);
    }
    idx += (c & 2) ? 2 : 0;
    const bool hi1 = (c & 1) != 0;
    const float send = hi1 ? x4[0] : x4[1];
    const float keep = hi1 ? x4[1] : x4[0];
    idx += (c & 1) ? 1 : 0;
    row = idx;
    return keep + __shfl_xor(send, 1, 64);
  } else {   // R == 4
    const bool hi2 = (c & 2) != 0;
    const float send = hi2 ? x2[0] : x2[1];
    const float keep = hi2 ? x2[1] : x2[0];
    idx += (c & 2) ? 1 : 0;
    row = idx;
    const float s = keep + __shfl_xor(send, 2, 64);
    return s + __shfl_xor(s, 1, 64);
  }
}

template <int DH, int T>
struct BwdSmem {
  float gq[T][DH / 8][DH];   // per step, per wave: dq partial sums over the wave's columns
  float gk[T][DH / 8][DH];
  float ga[T][DH];           // per step, per column: dalpha, dbeta terms
  float gb[T][DH];
};

template <typename InT, int DH, int T>
__global__ __launch_bounds__(64 * (DH / 8)) void gdn_bwd_kernel(
    const float* __restrict__ dy, const float* __restrict__ dfinal, const InT* __restrict__ q,
    const InT* __restrict__ k, const InT* __restrict__ v, const InT* __restrict__ alpha, const InT* __restrict__ beta,
    const float* __restrict__ h0, const float* __restrict__ ckpt, InT* __restrict__ dq, InT* __restrict__ dk,
    InT* __restrict__ dv, InT* __restrict__ dalpha, InT* __restrict__ dbeta, float* __restrict__ dh0, int H, int L,
    int nC) {
  constexpr int R = DH / 8, NW = DH / 8, NG = T / kU;
  __shared__ BwdSmem<DH, T> sm;
  const int bh = blockIdx.x, b = bh / H, h = bh % H;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = lane & 7, j = 8 * w + c, i0 = R * (lane >> 3);
  const bool lead = (lane >> 3) == 0;   // one lane per column writes the per-column results
  float adj[R];
#pragma unroll
  for (int r = 0; r < R; ++r) adj[r] = dfinal != nullptr ? dfinal[((int64_t)bh * DH + i0 + r) * DH + j] : 0.f;
  for (int cc = nC - 1; cc >= 0; --cc) {
    const int t0 = cc * T;
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
      for (int g = 0; g < NG; ++g) {
#pragma unroll
        for (int r = 0; r < R; ++r) Sg[g][r] = S[r];
        if (g + 1 < NG) {
#pragma unroll
          for (int u = 0; u < kU; ++u) {
            const int64_t row = ((int64_t)b * L + t0 + kU * g + u) * H + h;
            step<InT, R, false>(S, load_step<InT, R, false>(q, k, v, alpha, beta, row, DH, i0, j));
          }
        }
      }
    }
    // level 2: each group recomputed into registers, then swept backwards
#pragma unroll
    for (int g = NG - 1; g >= 0; --g) {
      float St[kU][R];
      StepIn<InT, R, true> in[kU];
      float pv[kU];
      {
        float S[R];
#pragma unroll
        for (int r = 0; r < R; ++r) S[r] = Sg[g][r];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int64_t row = ((int64_t)b * L + t0 + kU * g + u) * H + h;
          in[u] = load_step<InT, R, true>(q, k, v, alpha, beta, row, DH, i0, j);
          pv[u] = step<InT, R, true>(S, in[u]);
#pragma unroll
          for (int r = 0; r < R; ++r) St[u][r] = S[r];
        }
      }
#pragma unroll
      for (int u = kU - 1; u >= 0; --u) {
        const int tl = kU * g + u;   // step within the interval
        const int64_t row = ((int64_t)b * L + t0 + tl) * H + h;
        const float go = dy[row * DH + j];
        const float a = in[u].a, bb = in[u].b, p = pv[u];
        float gq[R], gk[R];
        float d = 0.f, sa = 0.f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          adj[r] += in[u].q[r] * go;                      // dS += q go^T           (B0)
          gq[r] = St[u][r] * go;                           // dq = S_t go            (Bq)
          d += in[u].k[r] * adj[r];
        }
        d = col_sum(d);                                    // d_j = k^T dS
        const float wk = bb * in[u].v - a * bb * p, ad = a * bb * d;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float sp = u > 0 ? St[u - 1][r] : Sg[g][r];   // S_{t-1}
          gk[r] = adj[r] * wk - sp * ad;                   // dk terms A + B
          sa += adj[r] * sp;
        }
        sa = col_sum(sa);                                  // <dS, S_{t-1}> over this column
        if (lead) {
          rr::st(dv, row * DH + j, bb * d);                // dv = beta d            (Bv)
          sm.ga[tl][j] = sa - bb * d * p;                  // dalpha terms of this column
          sm.gb[tl][j] = d * (in[u].v - a * p);            // dbeta terms            (Bbeta)
        }
        int rq, rk;
        const float sq = col_reduce_scatter<R>(gq, lane, rq);
        const float sk = col_reduce_scatter<R>(gk, lane, rk);
        sm.gq[tl][w][i0 + rq] = sq;
        sm.gk[tl][w][i0 + rk] = sk;
#pragma unroll
        for (int r = 0; r < R; ++r) adj[r] = a * (adj[r] - bb * in[u].k[r] * d);   // (Bp')
      }
    }
    __syncthreads();
    // the interval's sums over the waves (dq, dk) and the columns (dalpha, dbeta), in order
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
      for (int jj = 0; jj < DH; ++jj) {
        sa += sm.ga[tl][jj];
        sb += sm.gb[tl][jj];
      }
      const int64_t row = ((int64_t)b * L + t0 + tl) * H + h;
      rr::st(dalpha, row, sa);
      rr::st(dbeta, row, sb);
    }
    __syncthreads();   // the next interval rewrites the sums
  }
  if (dh0 != nullptr) {
#pragma unroll
    for (int r = 0; r < R; ++r) dh0[((int64_t)bh * DH + i0 + r) * DH + j] = adj[r];
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
  if (B * H >= ((int64_t)1 << 31) || B * L * H * Dh >= ((int64_t)1 << 40))
    return rr::fail(RR_EUNSUPPORTED, std::string(who) + ": tensors too large");
  return RR_OK;
}

template <typename InT, int DH, int T>
void launch_bwd_t(const float* dy, const float* dfinal, const void* q, const void* k, const void* v, const void* alpha,
                  const void* beta, const float* h0, const float* ckpt, void* dq, void* dk, void* dv, void* dalpha,
                  void* dbeta, float* dh0, int64_t B, int64_t H, int64_t L, int64_t nC, hipStream_t s) {
  hipLaunchKernelGGL((gdn_bwd_kernel<InT, DH, T>), dim3((unsigned)(B * H)), dim3(64 * (DH / 8)), 0, s, dy, dfinal,
                     static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(v),
                     static_cast<const InT*>(alpha), static_cast<const InT*>(beta), h0, ckpt, static_cast<InT*>(dq),
                     static_cast<InT*>(dk), static_cast<InT*>(dv), static_cast<InT*>(dalpha), static_cast<InT*>(dbeta),
                     dh0, (int)H, (int)L, (int)nC);
}

template <typename InT, int DH>
void launch_bwd_dh(int64_t T, const float* dy, const float* dfinal, const void* q, const void* k, const void* v,
                   const void* alpha, const void* beta, const float* h0, const float* ckpt, void* dq, void* dk,
                   void* dv, void* dalpha, void* dbeta, float* dh0, int64_t B, int64_t H, int64_t L, int64_t nC,
                   hipStream_t s) {
  if (T == 32)
    launch_bwd_t<InT, DH, 32>(dy, dfinal, q, k, v, alpha, beta, h0, ckpt, dq, dk, dv, dalpha, dbeta, dh0, B, H, L, nC, s);
  else if (T == 16)
    launch_bwd_t<InT, DH, 16>(dy, dfinal, q, k, v, alpha, beta, h0, ckpt, dq, dk, dv, dalpha, dbeta, dh0, B, H, L, nC, s);
  else
    launch_bwd_t<InT, DH, 8>(dy, dfinal, q, k, v, alpha, beta, h0, ckpt, dq, dk, dv, dalpha, dbeta, dh0, B, H, L, nC, s);
}

}  // namespace

extern "C" int rr_gdn_fwd(const void* q, const void* k, const void* v, const void* alpha, const void* beta, int dtype,
                          int64_t B, int64_t L, int64_t H, int64_t Dh, int64_t seg, const float* h0, float* y,
                          float* ckpt, void* stream) {
  if (int rc = check_gdn("gdn_fwd", B, L, H, Dh, seg, dtype)) return rc;
  if (!q || !k || !v || !alpha || !beta || !y || !ckpt) return rr::fail(RR_EINVAL, "gdn_fwd: null pointer argument");
  const int64_t T = rr::chunk_len(L, seg), nC = L / T;
  hipStream_t s = static_cast<hipStream_t>(stream);
  RR_DISPATCH_DTYPE(dtype, {
    if (Dh == 64)
      hipLaunchKernelGGL((gdn_fwd_kernel<InT, 64>), dim3((unsigned)(B * H)), dim3(512), 0, s,
                         static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(v),
                         static_cast<const InT*>(alpha), static_cast<const InT*>(beta), h0, y, ckpt, (int)H, (int)L,
                         (int)T, (int)nC);
    else
      hipLaunchKernelGGL((gdn_fwd_kernel<InT, 32>), dim3((unsigned)(B * H)), dim3(256), 0, s,
                         static_cast<const InT*>(q), static_cast<const InT*>(k), static_cast<const InT*>(v),
                         static_cast<const InT*>(alpha), static_cast<const InT*>(beta), h0, y, ckpt, (int)H, (int)L,
                         (int)T, (int)nC);
  });
  return rr::check_launch("rr_gdn_fwd");
}

extern "C" int rr_gdn_bwd(const float* dy, const float* dfinal, const void* q, const void* k, const void* v,
                          const void* alpha, const void* beta, int dtype, int64_t B, int64_t L, int64_t H, int64_t Dh,
                          int64_t seg, const float* h0, const float* ckpt, void* dq, void* dk, void* dv,
                          void* dalpha, void* dbeta, float* dh0, void* stream) {
  if (int rc = check_gdn("gdn_bwd", B, L, H, Dh, seg, dtype)) return rc;
  if (!dy || !q || !k || !v || !alpha || !beta || !ckpt || !dq || !dk || !dv || !dalpha || !dbeta)
    return rr::fail(RR_EINVAL, "gdn_bwd: null pointer argument");
  const int64_t T = rr::chunk_len(L, seg), nC = L / T;
  hipStream_t s = static_cast<hipStream_t>(stream);
  RR_DISPATCH_DTYPE(dtype, {
    if (Dh == 64)
      launch_bwd_dh<InT, 64>(T, dy, dfinal, q, k, v, alpha, beta, h0, ckpt, dq, dk, dv, dalpha, dbeta, dh0, B, H, L,
                             nC, s);
    else
      launch_bwd_dh<InT, 32>(T, dy, dfinal, q, k, v, alpha, beta, h0, ckpt, dq, dk, dv, dalpha, dbeta, dh0, B, H, L,
                             nC, s);
  });
  return rr::check_launch("rr_gdn_bwd");
}
