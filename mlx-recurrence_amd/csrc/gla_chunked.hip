// gla_chunked.hip — GLA scan on bf16 MFMA (the chunked form of rr_chunked.h).
//
// GLA (reference gla.py:78-100) is the chunked recurrence of rr_chunked.h with
// u = v, B = k, C = q, d = j (value index), n = i (key index), per-step decay
// g_t and input weight 1.  The forward runs the shared pipelined kernels
// (chunk aggregates, state pass, one workgroup per chunk).  This file holds
// the backward's per-chunk kernel.
//
// Backward, per 32-step chunk (reference adjoint gla.py:184-236 in matrix
// form), with h_in the chunk's entering state (forward checkpoint), lam the
// adjoint of the chunk's last state flowing in from later chunks (from
// pass_kernel), M[t, s] = g_{s+1} ... g_t, gam_t = g_0 ... g_t, m31_t = M[31, t]:
//   CB = Q K^T, G2 = dY V^T, GH = dY h_in, UL = V lam, P = M o CB, MG = M o G2
//   dv = P^T dY + diag(m31) K lam^T
//   dk = MG^T Q + diag(m31) UL
//   dq = diag(gam) GH + MG K
//   dg_t = sum_{j,i} lam_t h_{t-1}
//        = sum_{r >= t} M'[r, t] F_t[r],   r = 0..32,
// where rows r < 32 are the chunk's steps and row 32 stands for lam:
//   M'[r, t] = M[r, t] (r < 32), m31_t (r = 32);
//   F_0[r] = X_r (r < 32), tr (r = 32);  F_{t+1}[r] = g_t F_t[r] + E'[r, t];
//   E'[r, s] = CB[r, s] G2[r, s] (r < 32), Y_s (r = 32);
//   X = rowsum(GH o Q), Y = rowsum(UL o K), tr = sum(lam o h_in).
// (F_t[r] collects the state h_{t-1} seen from row r, so no gate is ever
// divided by and zero or negative gates are exact.)
#include "rr_chunked.h"

namespace {

using rr::bf_split;
using rr::bf_val;
using rr::f32x16_t;
using rr::f32x4_t;
using rr::frag;
using rr::frag4;
using rr::mfma16;
using rr::mfma16k16;
using rr::mfma32;
using rr::u16x4_t;
using rr::u16x8_t;
using rr::chunked::PQ;
using rr::chunked::Q;
using rr::chunked::r32row;

// LDS of the backward kernel.  The operands that die after phase B1 (x) share
// space with the masked products written in phase B2 (y).
template <int D>
struct alignas(16) GlaBwdSmem {
  static constexpr int PD = D + 8;
  uint16_t Kn[Q][PD];                    // k   [s][i]
  uint16_t Qn[Q][PD];                    // q   [t][i]
  uint16_t KT[D][PQ];                    // k^T [i][s]
  uint16_t QT[D][PQ];                    // q^T [i][t]
  uint16_t GYT_hi[D][PQ], GYT_lo[D][PQ]; // dY^T [j][t]
  uint16_t LM_hi[D][PD], LM_lo[D][PD];   // lam [j][i]
  union {
    struct {                             // phase A -> B1
      uint16_t V[Q][PD];                     // v  [s][j]
      uint16_t GY_hi[Q][PD], GY_lo[Q][PD];   // dY [t][j]
    } x;
    struct {                             // phase B2 -> C
      uint16_t PT_hi[Q][PQ], PT_lo[Q][PQ];   // P^T  [s][t']
      uint16_t MGT_hi[Q][PQ], MGT_lo[Q][PQ]; // MG^T [s][t']
      uint16_t MG_hi[Q][PQ], MG_lo[Q][PQ];   // MG   [t'][s]
    } y;
  };
  float CB[Q][Q + 1];
  float G2[Q][Q + 1];
  float Cc[Q + 1][Q + 1];                // dg contributions M'[r, t] F_t[r]
  float XYp[4][2][Q];                    // per-wave partial X, Y
  float g[Q], gam[Q], m31[Q];
  float trw[4];
};

// Work split (4 waves).  The state tile [j][i] is cut into 16x16 blocks; wave
// w owns the column blocks nb = w, w + 4, ... (all row blocks db), holding
// h_in and lam of those blocks in registers, where they are directly the B
// operands of 16x16x16 MFMAs contracting over j: so each wave forms
// GH = dY h_in and UL = V lam for its columns in registers and later writes
// dq and dk of the same columns.  dv row block db goes to wave (db + NBN) % 4.
template <int D, int MODE>
union GlaBwdShared {
  GlaBwdSmem<D> m;
};
template <int D>
union GlaBwdShared<D, rr::chunked::kDirect> {
  GlaBwdSmem<D> m;
  rr::chunked::DirectSmem<D, D, true> d;
};

// lam comes from pass_kernel (kPipe) or from the direct sum (kDirect); in the
// direct mode the workgroup of chunk 0 also writes the initial-state gradient
// dh0 = (gam o dY_0)^T Q_0 + gam_31 lam.
template <int D, int MODE>
__global__ __launch_bounds__(256, 2) void gla_bwd_kernel(rr::ChunkArgs p) {
  constexpr int NBN = D / 16, NBD = D / 16;
  constexpr int CPW = (NBN + 3) / 4;   // column blocks per wave
  __shared__ GlaBwdShared<D, MODE> smu;
  auto& m = smu.m;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const rr::chunked::ChunkId id = rr::chunked::chunk_id(p, false);
  if (!id.valid) return;
  const int c = id.c, h = id.h, b = id.b;
  const int64_t bh = (int64_t)b * p.H + h;
  const int64_t base = (((int64_t)b * p.L + (int64_t)c * Q) * p.H + h) * D;  // element (b, t0, h, 0)
  const int rs = p.H * D;                                                   // step stride (elements)
  const int l15 = lane & 15, l4 = lane >> 4;

  f32x4_t lam[CPW][NBD], hin[CPW][NBD];
  u16x4_t lam_hi[CPW][NBD], lam_lo[CPW][NBD], hin_hi[CPW][NBD], hin_lo[CPW][NBD];
  if constexpr (MODE == rr::chunked::kDirect) {
    const float gam_all = rr::chunked::direct_sum<D, D, true, true>(p, c, b, h, 0.f, smu.d);
    const float* dfb = p.dfinal != nullptr ? p.dfinal + bh * D * D : nullptr;
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = w + 4 * cc;
#pragma unroll
      for (int db = 0; db < NBD; ++db) {
        lam[cc][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (nb < NBN) {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            lam[cc][db][r] = rr::chunked::direct_value<D, D, true, true>(smu.d, gam_all, dfb, 16 * db + 4 * l4 + r,
                                                                         16 * nb + l15);
        }
      }
    }
    __syncthreads();   // the chunk below reuses the LDS of the sum
  }
  // ------------------------------------------------ A: stage (all loads first)
  {
    constexpr int UV = (Q * D / 8 + 255) / 256, GV = (Q * D / 4 + 255) / 256;
    u16x8_t vv[UV], kv[UV], qv[UV];
    float4 gv[GV];
    float xv = 1.f;
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + 256 * v, tl = (i / (D / 8)) & (Q - 1), d0 = 8 * (i % (D / 8));
      const bool ok = i < Q * D / 8;
      const int off = tl * rs + d0;
      vv[v] = ok ? *reinterpret_cast<const u16x8_t*>(p.u + base + off) : u16x8_t{};
      kv[v] = ok ? *reinterpret_cast<const u16x8_t*>(p.Bm + base + off) : u16x8_t{};
      qv[v] = ok ? *reinterpret_cast<const u16x8_t*>(p.Cm + base + off) : u16x8_t{};
    }
#pragma unroll
    for (int v = 0; v < GV; ++v) {
      const int i = tid + 256 * v, tl = (i / (D / 4)) & (Q - 1), d0 = 4 * (i % (D / 4));
      gv[v] = i < Q * D / 4 ? *reinterpret_cast<const float4*>(p.dy + base + tl * rs + d0)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (tid < Q) xv = bf_val(p.delta[(base / D) + tid * p.H]);
    const float* lsrc = MODE == rr::chunked::kPipe ? p.agg + (bh * p.nC + c) * D * D : nullptr;
    const float* hsrc = c > 0 ? p.ckpt + (bh * p.nC + c - 1) * D * D
                              : (p.h0 != nullptr ? p.h0 + bh * D * D : nullptr);
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = w + 4 * cc;
#pragma unroll
      for (int db = 0; db < NBD; ++db) {
        if constexpr (MODE == rr::chunked::kPipe) lam[cc][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        hin[cc][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if (nb < NBN) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int d = 16 * db + 4 * l4 + r, n = 16 * nb + l15;
            if constexpr (MODE == rr::chunked::kPipe) lam[cc][db][r] = lsrc[d * D + n];
            if (hsrc != nullptr) hin[cc][db][r] = hsrc[c > 0 ? d * D + n : rr::chunked::state_off<true, D, D>(d, n)];
          }
        }
      }
    }
    // LDS writes
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + 256 * v, tl = (i / (D / 8)) & (Q - 1), d0 = 8 * (i % (D / 8));
      if (i < Q * D / 8) {
        *reinterpret_cast<u16x8_t*>(&m.x.V[tl][d0]) = vv[v];
        *reinterpret_cast<u16x8_t*>(&m.Kn[tl][d0]) = kv[v];
        *reinterpret_cast<u16x8_t*>(&m.Qn[tl][d0]) = qv[v];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          m.KT[d0 + e][tl] = kv[v][e];
          m.QT[d0 + e][tl] = qv[v][e];
        }
      }
    }
#pragma unroll
    for (int v = 0; v < GV; ++v) {
      const int i = tid + 256 * v, tl = (i / (D / 4)) & (Q - 1), d0 = 4 * (i % (D / 4));
      if (i < Q * D / 4) {
        const float g4[4] = {gv[v].x, gv[v].y, gv[v].z, gv[v].w};
        u16x4_t hi4, lo4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint16_t hi, lo;
          bf_split(g4[e], hi, lo);
          hi4[e] = hi;
          lo4[e] = lo;
          m.GYT_hi[d0 + e][tl] = hi;
          m.GYT_lo[d0 + e][tl] = lo;
        }
        *reinterpret_cast<u16x4_t*>(&m.x.GY_hi[tl][d0]) = hi4;
        *reinterpret_cast<u16x4_t*>(&m.x.GY_lo[tl][d0]) = lo4;
      }
    }
    if (w == 0) {
      const rr::chunked::StepScalars sc = rr::chunked::step_scalars<true>(lane < Q ? xv : 1.f, 0.f, lane);
      if (lane < Q) {
        m.g[lane] = xv;
        m.gam[lane] = sc.gam;
        m.m31[lane] = sc.m31;
      }
    }
    float part = 0.f;
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = w + 4 * cc;
#pragma unroll
      for (int db = 0; db < NBD; ++db) {
        rr::bf_split4(lam[cc][db], lam_hi[cc][db], lam_lo[cc][db]);
        rr::bf_split4(hin[cc][db], hin_hi[cc][db], hin_lo[cc][db]);
        if (nb < NBN) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int d = 16 * db + 4 * l4 + r, n = 16 * nb + l15;
            m.LM_hi[d][n] = lam_hi[cc][db][r];
            m.LM_lo[d][n] = lam_lo[cc][db][r];
            part += lam[cc][db][r] * hin[cc][db][r];
          }
        }
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o);
    if (lane == 0) m.trw[w] = part;
  }
  __syncthreads();
  // ------------------------------------------------ B1: GH, UL (registers), CB, G2 (32x32)
  f32x4_t gh[CPW][2], ul[CPW][2];
#pragma unroll
  for (int cc = 0; cc < CPW; ++cc) {
    const int nb = w + 4 * cc;
    float xp[2][4] = {}, yp[2][4] = {};
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      gh[cc][tb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      ul[cc][tb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (nb < NBN) {
#pragma unroll
        for (int db = 0; db < NBD; ++db) {
          const int row = 16 * tb + l15, k0 = 16 * db + 4 * l4;
          const u16x4_t ah = frag4(&m.x.GY_hi[row][k0]), al = frag4(&m.x.GY_lo[row][k0]);
          const u16x4_t av = frag4(&m.x.V[row][k0]);
          gh[cc][tb] = mfma16k16(ah, hin_hi[cc][db], gh[cc][tb]);
          gh[cc][tb] = mfma16k16(ah, hin_lo[cc][db], gh[cc][tb]);
          gh[cc][tb] = mfma16k16(al, hin_hi[cc][db], gh[cc][tb]);
          ul[cc][tb] = mfma16k16(av, lam_hi[cc][db], ul[cc][tb]);
          ul[cc][tb] = mfma16k16(av, lam_lo[cc][db], ul[cc][tb]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tb + 4 * l4 + r, n = 16 * nb + l15;
          xp[tb][r] = gh[cc][tb][r] * bf_val(m.Qn[t][n]);
          yp[tb][r] = ul[cc][tb][r] * bf_val(m.Kn[t][n]);
        }
      }
    }
    // X, Y partials of this wave's columns: sum over the 16 lanes of a row group
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) {
          xp[tb][r] += __shfl_xor(xp[tb][r], o);
          yp[tb][r] += __shfl_xor(yp[tb][r], o);
        }
        if (l15 == 0) {
          const int t = 16 * tb + 4 * l4 + r;
          if (cc == 0) {
            m.XYp[w][0][t] = xp[tb][r];
            m.XYp[w][1][t] = yp[tb][r];
          } else {
            m.XYp[w][0][t] += xp[tb][r];
            m.XYp[w][1][t] += yp[tb][r];
          }
        }
      }
    }
  }
  f32x16_t cg = {};   // wave 0: CB = Q K^T; wave 1: G2 = dY V^T
  if (w == 0) {
#pragma unroll
    for (int kb = 0; kb < D / 16; ++kb)
      cg = mfma32(frag(&m.Qn[lane & 31][16 * kb + 8 * (lane >> 5)]),
                  frag(&m.Kn[lane & 31][16 * kb + 8 * (lane >> 5)]), cg);
#pragma unroll
    for (int r = 0; r < 16; ++r) m.CB[r32row(r, lane)][lane & 31] = cg[r];
  } else if (w == 1) {
#pragma unroll
    for (int kb = 0; kb < D / 16; ++kb) {
      const u16x8_t fb = frag(&m.x.V[lane & 31][16 * kb + 8 * (lane >> 5)]);
      cg = mfma32(frag(&m.x.GY_hi[lane & 31][16 * kb + 8 * (lane >> 5)]), fb, cg);
      cg = mfma32(frag(&m.x.GY_lo[lane & 31][16 * kb + 8 * (lane >> 5)]), fb, cg);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) m.G2[r32row(r, lane)][lane & 31] = cg[r];
  }
  __syncthreads();
  // ------------------------------------------------ B2: masked products; dg
  if (w != 2) {
    // wave 0: P^T (from its CB registers); wave 1: MG^T (from G2 registers);
    // wave 3: MG (from G2 in LDS)
    float md[16];
    rr::chunked::decay_block32<true>(m.g, 0.f, lane, md);
    const int s = lane & 31;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tp = r32row(r, lane);
      uint16_t hi, lo;
      if (w == 0) {
        bf_split(md[r] * cg[r], hi, lo);
        m.y.PT_hi[s][tp] = hi;
        m.y.PT_lo[s][tp] = lo;
      } else if (w == 1) {
        bf_split(md[r] * cg[r], hi, lo);
        m.y.MGT_hi[s][tp] = hi;
        m.y.MGT_lo[s][tp] = lo;
      } else {
        bf_split(md[r] * m.G2[tp][s], hi, lo);
        m.y.MG_hi[tp][s] = hi;
        m.y.MG_lo[tp][s] = lo;
      }
    }
  } else {
    if (lane <= Q) {
      const int row = lane;
      float e[Q], fv[Q];
      float f;
      if (row < Q) {
        f = m.XYp[0][0][row] + m.XYp[1][0][row] + m.XYp[2][0][row] + m.XYp[3][0][row];
#pragma unroll
        for (int s = 0; s < Q; ++s) e[s] = s < row ? m.CB[row][s] * m.G2[row][s] : 0.f;
      } else {
        f = m.trw[0] + m.trw[1] + m.trw[2] + m.trw[3];
#pragma unroll
        for (int s = 0; s < Q; ++s) e[s] = m.XYp[0][1][s] + m.XYp[1][1][s] + m.XYp[2][1][s] + m.XYp[3][1][s];
      }
#pragma unroll
      for (int t = 0; t < Q; ++t) {
        fv[t] = f;
        f = m.g[t] * f + e[t];
      }
      const int tmax = row < Q ? row : Q - 1;
      float mm = 1.f;
#pragma unroll
      for (int t = Q - 1; t >= 0; --t) {
        const bool act = t <= tmax;
        m.Cc[row][t] = act ? mm * fv[t] : 0.f;
        if (act) mm *= m.g[t];
      }
    }
    rr::wave_lds_sync();
    if (lane < Q) {
      float hp = 0.f;
#pragma unroll
      for (int r = 0; r <= Q; ++r) hp += m.Cc[r][lane];
      rr::st_bf16(p.ddelta, base / D + lane * p.H, hp);
    }
  }
  __syncthreads();
  // ------------------------------------------------ C: dv, dk, dq
  // dv row blocks db with (db + NBN) % 4 == w
#pragma unroll
  for (int db = 0; db < NBD; ++db) {
    if ((db + NBN) % 4 != w) continue;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      f32x4_t a1 = {0.f, 0.f, 0.f, 0.f}, a2 = {0.f, 0.f, 0.f, 0.f};
      {
        const int k0 = 8 * l4;
        const u16x8_t ph = frag(&m.y.PT_hi[16 * tb + l15][k0]), pl = frag(&m.y.PT_lo[16 * tb + l15][k0]);
        const u16x8_t gh8 = frag(&m.GYT_hi[16 * db + l15][k0]), gl8 = frag(&m.GYT_lo[16 * db + l15][k0]);
        a1 = mfma16(ph, gh8, a1);
        a1 = mfma16(ph, gl8, a1);
        a1 = mfma16(pl, gh8, a1);
      }
#pragma unroll
      for (int kk = 0; kk < D / 32; ++kk) {
        const int k0 = 32 * kk + 8 * l4;
        const u16x8_t fa = frag(&m.Kn[16 * tb + l15][k0]);
        a2 = mfma16(fa, frag(&m.LM_hi[16 * db + l15][k0]), a2);
        a2 = mfma16(fa, frag(&m.LM_lo[16 * db + l15][k0]), a2);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * tb + 4 * l4 + r;
        rr::st_bf16(p.du, base + t * rs + 16 * db + l15, a1[r] + m.m31[t] * a2[r]);
      }
    }
  }
  // dk, dq of this wave's columns
#pragma unroll
  for (int cc = 0; cc < CPW; ++cc) {
    const int nb = w + 4 * cc;
    if (nb >= NBN) continue;
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const int row = 16 * tb + l15, k0 = 8 * l4;
      f32x4_t ak = {0.f, 0.f, 0.f, 0.f}, aq = {0.f, 0.f, 0.f, 0.f};
      const u16x8_t fq = frag(&m.QT[16 * nb + l15][k0]);
      ak = mfma16(frag(&m.y.MGT_hi[row][k0]), fq, ak);
      ak = mfma16(frag(&m.y.MGT_lo[row][k0]), fq, ak);
      const u16x8_t fk = frag(&m.KT[16 * nb + l15][k0]);
      aq = mfma16(frag(&m.y.MG_hi[row][k0]), fk, aq);
      aq = mfma16(frag(&m.y.MG_lo[row][k0]), fk, aq);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * tb + 4 * l4 + r;
        const int64_t gi = base + t * rs + 16 * nb + l15;
        rr::st_bf16(p.dB, gi, ak[r] + m.m31[t] * ul[cc][tb][r]);
        rr::st_bf16(p.dC, gi, m.gam[t] * gh[cc][tb][r] + aq[r]);
      }
    }
  }
  if constexpr (MODE == rr::chunked::kDirect) {
    if (c == 0 && p.dh0 != nullptr) {
      // dh0 = (gam o dY_0)^T Q_0 + gam_31 lam, blocks of this wave's columns
      const float g31 = m.gam[Q - 1];
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        const int nb = w + 4 * cc;
        if (nb >= NBN) continue;
        const int k0 = 8 * l4;
        const u16x8_t qf = frag(&m.QT[16 * nb + l15][k0]);
        u16x8_t qh, ql;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          uint16_t hi, lo;
          bf_split(m.gam[k0 + e] * bf_val(qf[e]), hi, lo);
          qh[e] = hi;
          ql[e] = lo;
        }
#pragma unroll
        for (int db = 0; db < NBD; ++db) {
          const u16x8_t ah = frag(&m.GYT_hi[16 * db + l15][k0]), al = frag(&m.GYT_lo[16 * db + l15][k0]);
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
          acc = mfma16(ah, qh, acc);
          acc = mfma16(ah, ql, acc);
          acc = mfma16(al, qh, acc);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int d = 16 * db + 4 * l4 + r, n = 16 * nb + l15;
            p.dh0[bh * D * D + rr::chunked::state_off<true, D, D>(d, n)] = acc[r] + g31 * lam[cc][db][r];
          }
        }
      }
    }
  }
}

template <int D>
int launch_gla_fwd(const rr::ChunkArgs& p, int64_t B, hipStream_t s) {
  return rr::chunked::launch_fwd<D, D, true>(p, B, s);
}

template <int D>
int launch_gla_bwd(const rr::ChunkArgs& p, int64_t B, hipStream_t s) {
  if (p.mode == rr::chunked::kDirect) {
    if constexpr (D * D <= rr::chunked::kDirectMaxState) {
      hipLaunchKernelGGL((gla_bwd_kernel<D, rr::chunked::kDirect>), rr::chunked::chunk_grid(p), dim3(256), 0, s, p);
      return rr::check_launch("gla chunked backward");
    } else {
      return rr::fail(RR_EUNSUPPORTED, "gla chunked backward: state too large for the direct mode");
    }
  }
  hipLaunchKernelGGL((rr::chunked::agg_kernel<D, D, true>), rr::chunked::chunk_grid(p), dim3(64), 0, s, p, 1);
  if (int rc = rr::check_launch("gla chunked backward aggregates")) return rc;
  hipLaunchKernelGGL((rr::chunked::pass_kernel<D, D, true>), dim3(D * D / 256, p.H, (unsigned)B), dim3(256), 0, s,
                     p, 1);
  if (int rc = rr::check_launch("gla chunked backward adjoint pass")) return rc;
  hipLaunchKernelGGL((gla_bwd_kernel<D, rr::chunked::kPipe>), rr::chunked::chunk_grid(p), dim3(256), 0, s, p);
  return rr::check_launch("gla chunked backward");
}

int64_t align64(int64_t n) { return (n + 63) / 64 * 64; }

}  // namespace

namespace rr {

bool gla2_supported(int dtype, int64_t B, int64_t L, int64_t H, int64_t seg, int64_t Dh, int pass) {
  if (dtype != RR_BF16 || chunk_len(L, seg) != chunked::Q) return false;
  if ((L / chunked::Q) * ((B * H + chunked::kXcds - 1) / chunked::kXcds * chunked::kXcds) >= ((int64_t)1 << 31))
    return false;
  if (pass == 0) return Dh == 32 || Dh == 64 || Dh == 128;
  return Dh == 32 || Dh == 64;
}

int gla2_mode(int64_t nC, int64_t Dh) {
  return nC <= chunked::kDirectMaxChunks && Dh * Dh <= chunked::kDirectMaxState ? chunked::kDirect : chunked::kPipe;
}

size_t gla2_ws_bytes(int64_t B, int64_t H, int64_t nC, int64_t Dh, int pass) {
  if (gla2_mode(nC, Dh) == chunked::kDirect) return 0;
  int64_t f = align64(B * H * nC);
  if (pass == 1) f += align64(B * H * nC * Dh * Dh);
  return (size_t)f * sizeof(float);
}

void gla2_carve_ws(ChunkArgs& a, void* ws, int64_t B, int pass) {
  float* f = static_cast<float*>(ws);
  a.ws = a.tot = a.agg = nullptr;
  if (a.mode == chunked::kDirect) return;
  a.tot = f;
  f += align64(B * a.H * a.nC);
  a.agg = pass == 1 ? f : nullptr;
}

int gla2_fwd(const ChunkArgs& p, int64_t B, hipStream_t s) {
  switch (p.DH) {
    case 32: return launch_gla_fwd<32>(p, B, s);
    case 64: return launch_gla_fwd<64>(p, B, s);
    case 128: return launch_gla_fwd<128>(p, B, s);
    default: return fail(RR_EUNSUPPORTED, "gla chunked: unsupported Dh");
  }
}

int gla2_bwd(const ChunkArgs& p, int64_t B, hipStream_t s) {
  switch (p.DH) {
    case 32: return launch_gla_bwd<32>(p, B, s);
    case 64: return launch_gla_bwd<64>(p, B, s);
    default: return fail(RR_EUNSUPPORTED, "gla chunked backward: unsupported Dh");
  }
}

}  // namespace rr
