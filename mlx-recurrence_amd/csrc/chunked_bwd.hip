// chunked_bwd.hip — backward of the chunked scans (rr_chunked.h) with the
// state blocks owned by columns: GLA (any size) and SSD with N >= 64.
//
// Per 32-step chunk (reference adjoints ssd.py:203-268, gla.py:184-236 in
// matrix form), with h_in the state entering the chunk (forward checkpoint),
// lam the adjoint of the chunk's last state flowing in from later chunks,
// M[t, s] = dec_{s+1} ... dec_t, gam_t = dec_0 ... dec_t, m31_t = M[31, t],
// w_t the input weight (SSD delta_t, GLA 1) and rows d / columns n of the
// state (SSD channel / state, GLA j / i):
//   CB = C B^T, G2 = dY U^T, GH = dY h_in, UL = U lam, P = M o CB, MG = M o G2
//   du = diag(w) (P^T dY + diag(m31) B lam^T)
//   Z  = MG^T C + diag(m31) UL,  dB = diag(w) Z
//   dC = diag(gam) GH + (MG o w_s) B
//   Hp_t = sum_{d,n} lam_t h_{t-1}
//        = sum_{t'} (M o W)[t', t] + m31_t (P_t + gam_{t-1} tr),   W = E Mh + X gam_{t-1}
//          E = CB o G2 o w_s,  Mh[s, t] = M[t-1, s] (s < t, else 0),  P_t = sum_s Mh[s, t] Y_s
//          X = rowsum(GH o C), Y = rowsum(UL o B) o w, tr = sum(lam o h_in)
//        (lam_t and h_{t-1} factor through M[t', t] and M[t-1, s]: division free,
//        so zero or negative GLA gates are exact)
//   GLA: dg_t = Hp_t.
//   SSD: d(delta)_t = a dec_t Hp_t + sum_n B_t Z_t = a T_t + (1 - a delta_t) sum_n B_t Z_t
//        with T_t = sum_{d,n} lam_t h_t = R_t + sum_{t' >= t} gam X + sum_{s <= t} m31 w Y
//        + m31_t gam_t tr,  R_t = sum_{t' >= t, s <= t} (M o w_s o G2 o CB)[t', s]
//        (h_t and lam_t both expand without dividing by a decay), and per state n
//        dA[n] = sum_t C (K B) + sum_t gam cd C GH + sum_t m31 (cd_31 - cd) w B UL
//                + gam_31 cd_31 sum_d lam h_in,   K = M o w_s o G2 o (cd_t - cd_s)
//        (cd = in-chunk cumulative delta; from d exp(a (cd_t - cd_s)) / da)
//   lam_prev = (gam o dY)^T C + gam_31 lam   (adjoint handed to chunk c - 1)
// (derived from the per-step adjoint; checked against the float64 oracle).
//
// Work split (4 waves).  The state tile [d][n] is cut into 16x16 blocks; wave
// w owns the column blocks nb = w, w + 4, ... (all row blocks db) and holds
// h_in and lam of those blocks in registers, where a 16x16 accumulator block
// is directly the B operand of a 16x16x16 MFMA contracting over its rows: so
// each wave forms GH and UL of its columns in registers and writes dB and dC
// (and the dA of) those columns.  du row block db goes to wave (db + NBN) % 4
// (two blocks per wave with Dh = 128).
//
// Modes as in the forward: kWhole (a head per workgroup, lam carried in
// registers from chunk to chunk), kPipe (lam from pass_kernel), kDirect (lam
// from the direct sum; the workgroup of chunk 0 also forms dh0), kPair (a
// workgroup per run of R = 2 or 4 chunks, lam of the run's last chunk from
// the adjoint scan, which stores every R-th adjoint only; the workgroup forms
// the adjoint entering each earlier chunk of the run itself, in the layouts
// of both of its uses: the column blocks, lam_prev = gam_31 lam + (gam o
// dY)^T C, at the end of phase B1 while dY is staged, and du's operand rows,
// the same sum transposed, C^T diag(gam) dY, in phase C).
#include <type_traits>
#include <utility>

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
using rr::chunked::kDirect;
using rr::chunked::kPair;
using rr::chunked::kPipe;
using rr::chunked::kWhole;
using rr::chunked::PQ;
using rr::chunked::Q;
using rr::chunked::r32row;

// LDS of the backward kernel.  The operands that die after phase B1 (x) share
// space with the masked products written in phase B2 (y).  In the one-chunk
// modes (REG: kPipe, kDirect) the du operands dY^T and lam are register
// fragments (dY^T from global memory; lam from the pass's output, or from the
// direct sum's LDS before the chunk reuses it), so GYT and LM shrink to a row.
template <int DH, int NS, bool GLA, bool REG>
struct alignas(16) ColBwdSmem {
  static constexpr int PD = DH + 8, PN = NS + 8, TD = REG ? 1 : DH;
  uint16_t Kn[Q][PN];                      // B [s][n]
  uint16_t Qn[Q][PN];                      // C [t][n]
  uint16_t GYT_hi[TD][PQ], GYT_lo[TD][PQ]; // dY^T [d][t]
  uint16_t LM_hi[TD][PN], LM_lo[TD][PN];   // lam [d][n]
  union {
    struct {                               // phase A -> B1
      uint16_t V[Q][PD];                       // U [s][d]
      uint16_t GY_hi[Q][PD], GY_lo[Q][PD];     // dY [t][d]
    } x;
    struct {                               // phase B2 -> C
      uint16_t PT_hi[Q][PQ], PT_lo[Q][PQ];     // P^T        [s][t']
      uint16_t MGT_hi[Q][PQ], MGT_lo[Q][PQ];   // MG^T       [s][t']
      uint16_t MG_hi[Q][PQ], MG_lo[Q][PQ];     // MG o w_s   [t'][s]
      uint16_t Km_hi[GLA ? 1 : Q][PQ];         // SSD: K     [t'][s]
      uint16_t Km_lo[GLA ? 1 : Q][PQ];
    } y;
  };
  float CB[Q][Q + 1];
  float G2[Q][Q + 1];
  float XY[GLA ? 2 : 1][Q];                // GLA: X, Y (sums of the per-wave partials)
  float XYp[4][2][Q];                      // per-wave partial X, Y
  float BZp[GLA ? 1 : 4][Q];               // SSD: per-wave partial sum_n B Z
  float xin[Q], dec[Q], gam[Q], m31[Q], w[Q], cd[Q];
  float Rp[GLA ? 1 : 4][Q];                // SSD: per-wave partials of R_t (T_t = sum lam_t h_t)
  float Ts[GLA ? 1 : 2][Q];                // SSD: suffix of gam X, prefix of m31 w Y
  float trw[4];
};

template <int DH, int NS, int MODE, bool GLA>
union ColBwdShared {
  ColBwdSmem<DH, NS, GLA, MODE != kWhole> m;
};
// Wide states (past kDirectMaxState) in the direct mode: the adjoint summed by
// direct_sum_wide; du's row-owned operands of it go through the workspace
// (the pipelined mode's adjoint slots).
template <int DH, int NS>
constexpr bool kWideDirect = DH * NS > rr::chunked::kDirectMaxState;
template <int DH, int NS, bool GLA>
union ColBwdShared<DH, NS, kDirect, GLA> {
  ColBwdSmem<DH, NS, GLA, true> m;
  rr::chunked::DirectLds<DH, NS, true> d;
};

// Workgroups per CU the LDS allows (the register budget follows); SSD's
// direct mode for short sequences (few workgroups) keeps the registers of two.
template <int DH, int NS, int MODE, bool GLA>
constexpr int kColBwdWgs = MODE == kPair ? 2   // the carried du operands: the registers of two
                           : (int)(160 * 1024 / sizeof(ColBwdShared<DH, NS, MODE, GLA>)) >= 3 &&
                                     (GLA || MODE != kDirect || kWideDirect<DH, NS>)
                               ? 3
                           : (int)(160 * 1024 / sizeof(ColBwdShared<DH, NS, MODE, GLA>)) >= 2                          ? 2
                                                                                                                      : 1;

template <int DH, int NS, int MODE, bool GLA>
__global__ __launch_bounds__(256, (kColBwdWgs<DH, NS, MODE, GLA>)) void col_bwd_kernel(rr::ChunkArgs p) {
  constexpr int NBN = NS / 16, NBD = DH / 16;
  constexpr int CPW = (NBN + 3) / 4;   // column blocks per wave
  constexpr bool REG = MODE != kWhole;   // du operands as register fragments
  __shared__ ColBwdShared<DH, NS, MODE, GLA> smu;
  auto& m = smu.m;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  int h, b, cbeg, cend;
  if constexpr (MODE == kWhole) {
    h = blockIdx.y, b = blockIdx.z, cbeg = 0, cend = p.nC;
  } else if constexpr (MODE == kPair) {
    const rr::chunked::ChunkId id = rr::chunked::run_id(p);
    if (!id.valid) return;
    h = id.h, b = id.b, cbeg = p.R * id.c, cend = p.R * id.c + p.R;
  } else {
    // early chunks cost most where the adjoint is a sum over the later ones
    const rr::chunked::ChunkId id = rr::chunked::chunk_id(p, MODE == kDirect, false);
    if (!id.valid) return;
    h = id.h, b = id.b, cbeg = id.c, cend = id.c + 1;
  }
  const float a = rr::chunked::head_rate<GLA>(p, h);
  const int64_t bh = (int64_t)b * p.H + h;
  const int rsD = p.H * DH, rsN = p.H * NS;   // step strides (elements) of [.., H, DH] / [.., H, NS]
  const int l15 = lane & 15, l4 = lane >> 4;
  const int mydb = ((w - NBN) % 4 + 4) % 4;   // the first row block of du this wave forms
  constexpr int DPW = (NBD + 3) / 4;           // du row blocks per wave: mydb, mydb + 4, ...

  f32x4_t lam[CPW][NBD];
  float plm[REG && MODE != kPair ? DPW : 1][REG && MODE != kPair ? NS / 32 : 1][8];   // du operand: lam[16 (mydb + 4 k) + l15][32 kk + 8 l4 + e]
  // kPair's du operand: lam[16 (mydb + 4 k) + l15][16 nb + 4 l4 + r] (the layout
  // of the accumulator that carries it across the pair)
  f32x4_t plm4[MODE == kPair ? DPW : 1][MODE == kPair ? NBN : 1];
#pragma unroll
  for (int cc = 0; cc < CPW; ++cc)
#pragma unroll
    for (int db = 0; db < NBD; ++db) lam[cc][db] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // the chunk's inputs (phase A), loaded by `issue` at the start of the
  // chunk.  (Issued during the direct sum's reduction instead, they delay the
  // sum loops of the costliest workgroups more than they save: measured.)
  // Every load is issued by every thread, unconditionally and in bounds
  // (clamped indices; dropped values multiplied by 0, which the compiler
  // cannot turn into a branch around the load): a load under a branch makes
  // the branch's join wait for all of them.
  constexpr int UV = (Q * DH / 8 + 255) / 256, NV = (Q * NS / 8 + 255) / 256, GV = (Q * DH / 4 + 255) / 256;
  u16x8_t uv[UV], bv[NV], cv[NV];
  float4 gv[GV];
  float xv;
  f32x4_t hin[CPW][NBD];
  auto issue = [&](int c, int tid) {
    const int lane = tid & 63, l15 = lane & 15, l4 = lane >> 4;
    const int64_t row0 = (int64_t)b * p.L + (int64_t)c * Q;
    const int64_t baseD = (row0 * p.H + h) * DH, baseN = (row0 * p.H + h) * NS, baseX = row0 * p.H + h;
    // uniform chunk bases, 32-bit unsigned per-lane offsets
    const uint16_t* const uB = p.u + baseD;
    const uint16_t* const bB = p.Bm + baseN;
    const uint16_t* const cB = p.Cm + baseN;
    const float* const dyB = p.dy + baseD;
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + 256 * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
      uv[v] = rr::ld32<u16x8_t>(uB, (uint32_t)(tl * rsD + d0));
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const int i = tid + 256 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
      bv[v] = rr::ld32<u16x8_t>(bB, (uint32_t)(tl * rsN + n0));
      cv[v] = rr::ld32<u16x8_t>(cB, (uint32_t)(tl * rsN + n0));
    }
#pragma unroll
    for (int v = 0; v < GV; ++v) {
      const int i = tid + 256 * v, tl = (i / (DH / 4)) & (Q - 1), d0 = 4 * (i % (DH / 4));
      gv[v] = rr::ld32<float4>(dyB, (uint32_t)(tl * rsD + d0));
    }
    xv = bf_val(p.delta[baseX + (tid & (Q - 1)) * p.H]);   // only lanes < 32 of wave 0 use it
    // h_in: checkpoint slot c - 1 ([d][n]), h0 (state layout) or, with
    // neither, zero (the checkpoint buffer read and dropped; its values are finite)
    const float has_h = c > 0 || p.h0 != nullptr ? 1.f : 0.f;
    const auto hsrc = rr::as_global(c > 0 ? p.ckpt + (bh * p.nC + c - 1) * DH * NS
                                          : (p.h0 != nullptr ? p.h0 + bh * DH * NS : p.ckpt));
    const auto lsrc = rr::as_global(MODE == kPipe ? p.agg + rr::chunked::adj_slot(bh, p.nC, 1, c) * DH * NS : p.ckpt);
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = min(w + 4 * cc, NBN - 1);
      const float use = w + 4 * cc < NBN ? 1.f : 0.f;
#pragma unroll
      for (int db = 0; db < NBD; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 16 * db + 4 * l4 + r, n = 16 * nb + l15;
          if constexpr (MODE == kPipe) lam[cc][db][r] = use * rr::ld32<float>(lsrc, (uint32_t)(d * NS + n));
          hin[cc][db][r] =
              use * has_h * rr::ld32<float>(hsrc, (uint32_t)(c > 0 ? d * NS + n : rr::chunked::state_off<GLA, DH, NS>(d, n)));
        }
    }
  };
  if constexpr (MODE == kDirect && kWideDirect<DH, NS>) {
    // the adjoint leaving the chunk, this wave's column blocks (direct_sum_wide)
    const bool g0 = cbeg == 0 && p.dh0 != nullptr;   // uniform
    const float gam_all = rr::chunked::direct_sum_wide<DH, NS, GLA, true>(p, cbeg, b, h, a, smu.d, lam, g0);
    if (p.dfinal != nullptr) {
      const float* dfb = p.dfinal + bh * DH * NS;
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        if (w + 4 * cc < NBN) {
#pragma unroll
          for (int db = 0; db < NBD; ++db)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              lam[cc][db][r] +=
                  rr::chunked::direct_ext<DH, NS, GLA>(gam_all, dfb, 16 * db + 4 * l4 + r, 16 * (w + 4 * cc) + l15);
        }
      }
    }
    if (g0) {
      // dh0 = tot_0 lam(0) + G_0, G_0 = (gam o dY_0)^T C_0: chunk 0's step
      // scalars are range index 0 of the sum; the operands come straight
      // from memory (A: dY rows 8 (lane / 16) + e of column d; B: C rows of
      // column n)
      const float t0 = smu.d.tot[0];
      const int64_t row0 = (int64_t)b * p.L;
      float gw[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) gw[e] = smu.d.coef[0][8 * l4 + e];
      u16x8_t cfr[CPW];
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        const int nb = min(w + 4 * cc, NBN - 1);
#pragma unroll
        for (int e = 0; e < 8; ++e) cfr[cc][e] = p.Cm[((row0 + 8 * l4 + e) * p.H + h) * NS + 16 * nb + l15];
      }
#pragma unroll
      for (int db = 0; db < NBD; ++db) {
        float x[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = gw[e] * p.dy[((row0 + 8 * l4 + e) * p.H + h) * DH + 16 * db + l15];
        u16x8_t xh, xl;
        rr::bf_split8(x, xh, xl);
#pragma unroll
        for (int cc = 0; cc < CPW; ++cc) {
          if (w + 4 * cc < NBN) {
            f32x4_t g = {0.f, 0.f, 0.f, 0.f};
            g = mfma16(xh, cfr[cc], g);
            g = mfma16(xl, cfr[cc], g);
#pragma unroll
            for (int r = 0; r < 4; ++r)
              p.dh0[bh * DH * NS +
                    rr::chunked::state_off<GLA, DH, NS>(16 * db + 4 * l4 + r, 16 * (w + 4 * cc) + l15)] =
                  t0 * lam[cc][db][r] + g[r];
          }
        }
      }
    }
    // du's operands (rows mydb + 4 k of lam, every column: other waves'
    // blocks) are read in phase B2 as in the pipelined mode, from the
    // workspace slot of this chunk, written here
    float* lsl = p.agg + rr::chunked::adj_slot(bh, p.nC, 1, cbeg) * DH * NS;
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      if (w + 4 * cc < NBN) {
#pragma unroll
        for (int db = 0; db < NBD; ++db)
#pragma unroll
          for (int r = 0; r < 4; ++r) lsl[(16 * db + 4 * l4 + r) * NS + 16 * (w + 4 * cc) + l15] = lam[cc][db][r];
      }
    }
    __syncthreads();   // the chunk below reuses the LDS of the sum
  } else if constexpr (MODE == kDirect) {
    // the adjoint leaving the chunk; chunk 0's workgroup also stores dh0
    const float gam_all = rr::chunked::direct_sum<DH, NS, GLA, true, true>(p, cbeg, b, h, a, smu.d, p.dh0);
    const float* dfb = p.dfinal != nullptr ? p.dfinal + bh * DH * NS : nullptr;
    // lam of this wave's columns, and its du operands (rows of blocks mydb + 4 k)
    auto lam_at = [&](int cc, int db, int r) { return std::make_pair(16 * db + 4 * l4 + r, 16 * (w + 4 * cc) + l15); };
    auto plm_at = [&](int k, int kk, int e) {
      return std::make_pair(16 * (mydb + 4 * k) + l15, 32 * kk + 8 * l4 + e);
    };
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      if (w + 4 * cc < NBN) {
#pragma unroll
        for (int db = 0; db < NBD; ++db)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const auto [d, n] = lam_at(cc, db, r);
            lam[cc][db][r] = rr::chunked::direct_partial(smu.d, d, n);
          }
      }
    }
#pragma unroll
    for (int k = 0; k < DPW; ++k) {
      if (mydb + 4 * k < NBD) {
#pragma unroll
        for (int kk = 0; kk < NS / 32; ++kk)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const auto [d, n] = plm_at(k, kk, e);
            plm[k][kk][e] = rr::chunked::direct_partial(smu.d, d, n);
          }
      }
    }
    if (dfb != nullptr) {
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        if (w + 4 * cc < NBN) {
#pragma unroll
          for (int db = 0; db < NBD; ++db)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const auto [d, n] = lam_at(cc, db, r);
              lam[cc][db][r] += rr::chunked::direct_ext<DH, NS, GLA>(gam_all, dfb, d, n);
            }
        }
      }
#pragma unroll
      for (int k = 0; k < DPW; ++k) {
        if (mydb + 4 * k < NBD) {
#pragma unroll
          for (int kk = 0; kk < NS / 32; ++kk)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const auto [d, n] = plm_at(k, kk, e);
              plm[k][kk][e] += rr::chunked::direct_ext<DH, NS, GLA>(gam_all, dfb, d, n);
            }
        }
      }
    }
    __syncthreads();   // the chunk below reuses the LDS of the sum
  } else if constexpr (MODE == kWhole) {
    if (p.dfinal != nullptr) {
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        const int nb = w + 4 * cc;
        if (nb < NBN) {
#pragma unroll
          for (int db = 0; db < NBD; ++db)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              lam[cc][db][r] = p.dfinal[bh * DH * NS +
                                        rr::chunked::state_off<GLA, DH, NS>(16 * db + 4 * l4 + r, 16 * nb + l15)];
        }
      }
    }
  }
  // the adjoint handed to chunk c - 1 is needed for the whole head, and for dh0
  constexpr bool carry = MODE == kWhole;
  float dA_acc[CPW];   // SSD: dA of this lane's column (every l4 group holds the same sum)
#pragma unroll
  for (int cc = 0; cc < CPW; ++cc) dA_acc[cc] = 0.f;
  if constexpr (MODE == kPair) {
    // lam leaving the run (slot cbeg / R of the scan's output), this wave's column blocks
    const auto lsrc = rr::as_global(p.agg + rr::chunked::adj_slot(bh, p.nC, p.R, cbeg / p.R) * DH * NS);
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = min(w + 4 * cc, NBN - 1);
      const float use = w + 4 * cc < NBN ? 1.f : 0.f;
#pragma unroll
      for (int db = 0; db < NBD; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          lam[cc][db][r] = use * rr::ld32<float>(lsrc, (uint32_t)((16 * db + 4 * l4 + r) * NS + 16 * nb + l15));
    }
  }

  // One chunk.  kPair: LOAD for the run's last chunk (its adjoint from
  // memory), CARRY for every chunk but the run's first (it forms the adjoint
  // entering the chunk before it).  A lambda forced inline, so the loads and
  // carries are resolved at compile time (no branch around a load).
  auto chunk_body = [&](const int c, auto load_tag, auto carry_tag) __attribute__((always_inline)) {
    constexpr bool LOAD = decltype(load_tag)::value, CARRY = decltype(carry_tag)::value;
    // a fresh copy of the thread index per chunk keeps the compiler from
    // hoisting every per-lane LDS / global address of the body out of the loop
    int tidv = tid;
    asm volatile("" : "+v"(tidv));
    const int lane = tidv & 63, l15 = lane & 15, l4 = lane >> 4, tid = tidv;
    const int64_t row0 = (int64_t)b * p.L + (int64_t)c * Q;   // first (b, t) row of the chunk
    const int64_t baseD = (row0 * p.H + h) * DH, baseN = (row0 * p.H + h) * NS, baseX = row0 * p.H + h;
    uint16_t* const duB = p.du + baseD;
    uint16_t* const dBB = p.dB + baseN;
    uint16_t* const dCB = p.dC + baseN;
    float trn[CPW];   // SSD: sum over this lane's rows of lam o h_in, per column
    // ------------------------------------------------ A: stage
    {
      issue(c, tid);
      // LDS writes
#pragma unroll
      for (int v = 0; v < UV; ++v) {
        const int i = tid + 256 * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
        if (i < Q * DH / 8) *reinterpret_cast<u16x8_t*>(&m.x.V[tl][d0]) = uv[v];
      }
#pragma unroll
      for (int v = 0; v < NV; ++v) {
        const int i = tid + 256 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
        if (i < Q * NS / 8) {
          *reinterpret_cast<u16x8_t*>(&m.Kn[tl][n0]) = bv[v];
          *reinterpret_cast<u16x8_t*>(&m.Qn[tl][n0]) = cv[v];
        }
      }
#pragma unroll
      for (int v = 0; v < GV; ++v) {
        const int i = tid + 256 * v, tl = (i / (DH / 4)) & (Q - 1), d0 = 4 * (i % (DH / 4));
        if (i < Q * DH / 4) {
          const float g4[4] = {gv[v].x, gv[v].y, gv[v].z, gv[v].w};
          u16x4_t hi4, lo4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint16_t hi, lo;
            bf_split(g4[e], hi, lo);
            hi4[e] = hi;
            lo4[e] = lo;
            if constexpr (!REG) {
              m.GYT_hi[d0 + e][tl] = hi;
              m.GYT_lo[d0 + e][tl] = lo;
            }
          }
          *reinterpret_cast<u16x4_t*>(&m.x.GY_hi[tl][d0]) = hi4;
          *reinterpret_cast<u16x4_t*>(&m.x.GY_lo[tl][d0]) = lo4;
        }
      }
      if (w == 0) {
        const rr::chunked::StepScalars sc = rr::chunked::step_scalars<GLA>(lane < Q ? xv : (GLA ? 1.f : 0.f), a, lane);
        if (lane < Q) {
          m.xin[lane] = xv;
          m.dec[lane] = GLA ? xv : __expf(a * xv);
          m.gam[lane] = sc.gam;
          m.m31[lane] = sc.m31;
          m.w[lane] = sc.w;
          m.cd[lane] = sc.cd;
        }
      }
    }
    // sum lam o h_in per column (trn) and per wave (trw, read in phase B2);
    // whole head: with lam's LDS copy, before the barrier; register modes:
    // after it, so that the staging above does not wait for h_in (the
    // chunk's largest load)
    auto lam_hin = [&]() __attribute__((always_inline)) {
      float part = 0.f;
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        const int nb = w + 4 * cc;
        trn[cc] = 0.f;
        if (nb < NBN) {
#pragma unroll
          for (int db = 0; db < NBD; ++db) {
            u16x4_t hi4, lo4;
            rr::bf_split4(lam[cc][db], hi4, lo4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int d = 16 * db + 4 * l4 + r, n = 16 * nb + l15;
              if constexpr (!REG) {
                m.LM_hi[d][n] = hi4[r];
                m.LM_lo[d][n] = lo4[r];
              }
              trn[cc] += lam[cc][db][r] * hin[cc][db][r];
            }
          }
        }
        part += trn[cc];
        trn[cc] = rr::rows4_sum(trn[cc]);
      }
      part = rr::wave_sum(part);
      if (lane == 0) m.trw[w] = part;
    };
    if constexpr (!REG) lam_hin();
    __syncthreads();
    if constexpr (REG) lam_hin();
    // ------------------------------------------------ B1: GH, UL (registers), CB, G2 (32x32)
    f32x4_t gh[CPW][2], ul[CPW][2];
    float xs[2][4] = {}, ys[2][4] = {};   // this lane's shares of the row sums X, Y
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = w + 4 * cc;
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) gh[cc][tb] = ul[cc][tb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (nb >= NBN) continue;
#pragma unroll
      for (int db = 0; db < NBD; ++db) {
        u16x4_t hh, hl, lh, ll;
        rr::bf_split4(hin[cc][db], hh, hl);
        rr::bf_split4(lam[cc][db], lh, ll);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          const int row = 16 * tb + l15, k0 = 16 * db + 4 * l4;
          const u16x4_t ah = frag4(&m.x.GY_hi[row][k0]), al = frag4(&m.x.GY_lo[row][k0]);
          const u16x4_t av = frag4(&m.x.V[row][k0]);
          gh[cc][tb] = mfma16k16(ah, hh, gh[cc][tb]);
          gh[cc][tb] = mfma16k16(ah, hl, gh[cc][tb]);
          gh[cc][tb] = mfma16k16(al, hh, gh[cc][tb]);
          ul[cc][tb] = mfma16k16(av, lh, ul[cc][tb]);
          ul[cc][tb] = mfma16k16(av, ll, ul[cc][tb]);
        }
      }
#pragma unroll
      for (int tb = 0; tb < 2; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tb + 4 * l4 + r, n = 16 * nb + l15;
          xs[tb][r] += gh[cc][tb][r] * bf_val(m.Qn[t][n]);
          ys[tb][r] += ul[cc][tb][r] * bf_val(m.Kn[t][n]);
        }
    }
    // X, Y partials of this wave's columns: sums over the 16 lanes of a row group
#pragma unroll
    for (int tb = 0; tb < 2; ++tb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float xr = rr::row16_sum(xs[tb][r]), yr = rr::row16_sum(ys[tb][r]);
        if (l15 == 0) {
          const int t = 16 * tb + 4 * l4 + r;
          m.XYp[w][0][t] = xr;
          m.XYp[w][1][t] = yr;
        }
      }
    if constexpr (MODE == kPair && CARRY) {
      // the adjoint entering this chunk, for the run's chunk before it (lam is
      // dead here: UL above was its last use): lam <- gam_31 lam + (gam o dY)^T C,
      // dY^T [d][t] by transposing reads of the staged dY, (gam o C) [t][n]
      const float g31 = m.gam[Q - 1];
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        const int nb = w + 4 * cc;
        if (nb >= NBN) continue;
        const u16x8_t qf = rr::frag_tr(&m.Qn[0][16 * nb], ColBwdSmem<DH, NS, GLA, REG>::PN, lane);
        float qw[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) qw[e] = m.gam[8 * l4 + e] * bf_val(qf[e]);
        u16x8_t qh, ql;
        rr::bf_split8(qw, qh, ql);
#pragma unroll
        for (int db = 0; db < NBD; ++db) {
          constexpr int PD = ColBwdSmem<DH, NS, GLA, REG>::PD;
          const u16x8_t ah = rr::frag_tr(&m.x.GY_hi[0][16 * db], PD, lane);
          const u16x8_t al = rr::frag_tr(&m.x.GY_lo[0][16 * db], PD, lane);
          // all four hi / lo products: both factors are split fp32 values, and
          // the carried adjoint keeps the scan's 2^-17 relative accuracy
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
          acc = mfma16(al, ql, acc);
          acc = mfma16(ah, ql, acc);
          acc = mfma16(al, qh, acc);
          acc = mfma16(ah, qh, acc);
          lam[cc][db] = acc + g31 * lam[cc][db];
        }
      }
    }
    f32x16_t cg = {};   // wave 0: CB = C B^T; wave 1: G2 = dY U^T
    if (w == 0) {
#pragma unroll
      for (int kb = 0; kb < NS / 16; ++kb)
        cg = mfma32(frag(&m.Qn[lane & 31][16 * kb + 8 * (lane >> 5)]),
                    frag(&m.Kn[lane & 31][16 * kb + 8 * (lane >> 5)]), cg);
#pragma unroll
      for (int r = 0; r < 16; ++r) m.CB[r32row(r, lane)][lane & 31] = cg[r];
    } else if (w == 1) {
#pragma unroll
      for (int kb = 0; kb < DH / 16; ++kb) {
        const u16x8_t fb = frag(&m.x.V[lane & 31][16 * kb + 8 * (lane >> 5)]);
        cg = mfma32(frag(&m.x.GY_hi[lane & 31][16 * kb + 8 * (lane >> 5)]), fb, cg);
        cg = mfma32(frag(&m.x.GY_lo[lane & 31][16 * kb + 8 * (lane >> 5)]), fb, cg);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) m.G2[r32row(r, lane)][lane & 31] = cg[r];
    }
    __syncthreads();
    // ------------------------------------------------ B2: masked products; GLA dg / SSD T
    // one-chunk modes: this wave's du operands (row blocks mydb + 4 k), used
    // in phase C; the loads land while B2 runs (issued by every wave, clamped:
    // no branch join waits for them)
    float pdy[REG ? DPW : 1][REG ? 8 : 1];
    if constexpr (REG) {
#pragma unroll
      for (int k = 0; k < DPW; ++k) {
        const int d = 16 * min(mydb + 4 * k, NBD - 1) + l15;
#pragma unroll
        for (int e = 0; e < 8; ++e) pdy[k][e] = rr::ld32<float>(p.dy + baseD, (uint32_t)((8 * l4 + e) * rsD + d));
      }
    }
    if constexpr (MODE == kPair && LOAD) {
#pragma unroll
      for (int k = 0; k < DPW; ++k) {
        const int d = 16 * min(mydb + 4 * k, NBD - 1) + l15;
        const float* lsrc = p.agg + (rr::chunked::adj_slot(bh, p.nC, p.R, cbeg / p.R) * DH + d) * NS + 4 * l4;
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          const float4 l0 = *reinterpret_cast<const float4*>(lsrc + 16 * nb);
          plm4[k][nb] = f32x4_t{l0.x, l0.y, l0.z, l0.w};
        }
      }
    }
    if constexpr (MODE == kPipe || (MODE == kDirect && kWideDirect<DH, NS>)) {
#pragma unroll
      for (int k = 0; k < DPW; ++k) {
        const int d = 16 * min(mydb + 4 * k, NBD - 1) + l15;
        const float* lsrc = p.agg + (rr::chunked::adj_slot(bh, p.nC, 1, c) * DH + d) * NS + 8 * l4;
#pragma unroll
        for (int kk = 0; kk < NS / 32; ++kk) {
          const float4 l0 = *reinterpret_cast<const float4*>(lsrc + 32 * kk);
          const float4 l1 = *reinterpret_cast<const float4*>(lsrc + 32 * kk + 4);
          plm[k][kk][0] = l0.x, plm[k][kk][1] = l0.y, plm[k][kk][2] = l0.z, plm[k][kk][3] = l0.w;
          plm[k][kk][4] = l1.x, plm[k][kk][5] = l1.y, plm[k][kk][6] = l1.z, plm[k][kk][7] = l1.w;
        }
      }
    }
    if constexpr (!GLA) {
      // Wave w forms rows t' = t0 + q, q < 4, t0 = 8 w + 4 (lane / 32), of
      // every 32 x 32 product, column s = lane % 32 (one decay per element):
      // P^T and MG^T [s][t'] (four consecutive t': one 8-byte write each),
      // MG o w_s and K = MG o w_s o (cd_t' - cd_s) [t'][s], and its partial of
      // R_t = sum_{t' >= t} sum_{s <= t} (M o w_s o G2 o CB)[t', s] (prefix
      // over s along the lanes, then the rows t' >= s of column s).
      const int s = lane & 31, t0 = 8 * w + 4 * (lane >> 5);
      const float cds = m.cd[s], wsv = m.w[s];
      float pt[4], mg[4], rs = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int tp = t0 + q;
        const float ctp = m.cd[tp];
        const float md = rr::chunked::masked_exp(s <= tp, a * (ctp - cds));
        const float cb = m.CB[tp][s];
        pt[q] = md * cb;
        mg[q] = md * m.G2[tp][s];
        const float mgw = mg[q] * wsv;
        uint16_t hi, lo;
        bf_split(mgw, hi, lo);
        m.y.MG_hi[tp][s] = hi;
        m.y.MG_lo[tp][s] = lo;
        bf_split(mgw * (ctp - cds), hi, lo);
        m.y.Km_hi[tp][s] = hi;
        m.y.Km_lo[tp][s] = lo;
        const float k = rr::prefix32_sum(mgw * cb);
        rs += tp >= s ? k : 0.f;
      }
      u16x4_t hi4, lo4;
      rr::bf_split4(f32x4_t{pt[0], pt[1], pt[2], pt[3]}, hi4, lo4);
      *reinterpret_cast<u16x4_t*>(&m.y.PT_hi[s][t0]) = hi4;
      *reinterpret_cast<u16x4_t*>(&m.y.PT_lo[s][t0]) = lo4;
      rr::bf_split4(f32x4_t{mg[0], mg[1], mg[2], mg[3]}, hi4, lo4);
      *reinterpret_cast<u16x4_t*>(&m.y.MGT_hi[s][t0]) = hi4;
      *reinterpret_cast<u16x4_t*>(&m.y.MGT_lo[s][t0]) = lo4;
      rs = rr::halves_sum(rs);
      if (lane < Q) m.Rp[w][lane] = rs;
      if (w == 2) {
        // lanes 0..31: suffix of gam X in reversed lane order; lanes 32..63: prefix of m31 w Y
        const int tq = lane < Q ? Q - 1 - lane : lane - Q;
        // (every lane reads both factors and selects: no divergent branch)
        const int kx = lane < Q ? 0 : 1;
        const float gq = m.gam[tq], mw = m.m31[tq] * m.w[tq];
        const float xy =
            (lane < Q ? gq : mw) * (m.XYp[0][kx][tq] + m.XYp[1][kx][tq] + m.XYp[2][kx][tq] + m.XYp[3][kx][tq]);
        m.Ts[lane < Q ? 0 : 1][tq] = rr::prefix32_sum(xy);
      }
    } else if (w != 2) {
      // GLA: wave 0: P^T (CB registers); wave 1: MG^T (G2 registers); wave 3: MG o w_s
      float md[16];
      rr::chunked::decay_block32<true>(m.xin, a, lane, md);
      const int s = lane & 31;
      if (w != 3) {
        // rows r32row(4g .. 4g + 3) are consecutive: one 8-byte write per group
        uint16_t(*dst_hi)[PQ] = w == 0 ? m.y.PT_hi : m.y.MGT_hi;
        uint16_t(*dst_lo)[PQ] = w == 0 ? m.y.PT_lo : m.y.MGT_lo;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u16x4_t hi4, lo4;
          rr::bf_split4(f32x4_t{md[4 * g] * cg[4 * g], md[4 * g + 1] * cg[4 * g + 1], md[4 * g + 2] * cg[4 * g + 2],
                                md[4 * g + 3] * cg[4 * g + 3]},
                        hi4, lo4);
          const int tp = r32row(4 * g, lane);
          *reinterpret_cast<u16x4_t*>(&dst_hi[s][tp]) = hi4;
          *reinterpret_cast<u16x4_t*>(&dst_lo[s][tp]) = lo4;
        }
      } else {
        const float wsv = m.w[s];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int tp = r32row(r, lane);
          uint16_t hi, lo;
          const float mgw = md[r] * m.G2[tp][s] * wsv;
          bf_split(mgw, hi, lo);
          m.y.MG_hi[tp][s] = hi;
          m.y.MG_lo[tp][s] = lo;
        }
      }
    } else {
      // GLA: dg_t = sum_{t'} (M o W)[t', t] + m31_t (P_t + gam_{t-1} tr), division free:
      //   W = E Mh + X gam_{t-1},  E = CB o G2,  Mh[s, t] = M[t-1, s] = g_{s+1} ... g_{t-1} (s < t),
      //   P_t = sum_{s<t} Mh[s, t] Y_s
      // (E Mh on MFMA: lane holds column t = lane % 32 of Mh for s = 16 kb + 8 (lane / 32) + e)
      const int t = lane & 31, hf = lane >> 5;
      if (lane < Q) {
        m.XY[0][lane] = m.XYp[0][0][lane] + m.XYp[1][0][lane] + m.XYp[2][0][lane] + m.XYp[3][0][lane];
        m.XY[1][lane] = m.XYp[0][1][lane] + m.XYp[1][1][lane] + m.XYp[2][1][lane] + m.XYp[3][1][lane];
      }
      float mh[2][8];
      {
        float run = 1.f;
#pragma unroll
        for (int s = Q - 1; s >= 0; --s) {
          const float g = m.xin[(s + 1) & (Q - 1)];   // read in every lane (no branch around it)
          run = s == t - 1 ? 1.f : run * g;
          if (((s >> 3) & 1) == hf) mh[s >> 4][s & 7] = s < t ? run : 0.f;
        }
      }
      f32x16_t acc = {};
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        float ev[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int sv = 16 * kb + 8 * hf + e;
          ev[e] = m.CB[t][sv] * m.G2[t][sv];
        }
        u16x8_t eh, el, bh, bl;
        rr::bf_split8(ev, eh, el);
        rr::bf_split8(mh[kb], bh, bl);
        acc = mfma32(eh, bh, acc);
        acc = mfma32(eh, bl, acc);
        acc = mfma32(el, bh, acc);
      }
      rr::wave_lds_sync();   // XY
      float md[16];
      rr::chunked::decay_block32<true>(m.xin, 0.f, lane, md);
      const float gp = m.gam[(t + Q - 1) & (Q - 1)];
      const float gprev = t > 0 ? gp : 1.f;
      float cs = 0.f, ps = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) cs += md[r] * (acc[r] + m.XY[0][r32row(r, lane)] * gprev);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int e = 0; e < 8; ++e) ps += mh[kb][e] * m.XY[1][16 * kb + 8 * hf + e];
      cs = rr::halves_sum(cs);
      ps = rr::halves_sum(ps);
      if (lane < Q) {
        const float tr = m.trw[0] + m.trw[1] + m.trw[2] + m.trw[3];
        rr::st_bf16(p.ddelta, baseX + lane * p.H, cs + m.m31[lane] * (ps + gprev * tr));
      }
    }
    __syncthreads();
    // ------------------------------------------------ C: du, dB, dC (+ SSD dA terms, lam_prev)
#pragma unroll
    for (int k = 0; k < DPW; ++k) {
      const int db = mydb + 4 * k;
      if (db >= NBD) continue;
      u16x8_t gh8, gl8;   // dY^T fragment [t' = 8 l4 + e][d]
      if constexpr (REG) {
        rr::bf_split8(pdy[k], gh8, gl8);
      } else {
        gh8 = frag(&m.GYT_hi[16 * db + l15][8 * l4]);
        gl8 = frag(&m.GYT_lo[16 * db + l15][8 * l4]);
      }
      u16x8_t lh8[NS / 32], ll8[NS / 32];   // lam fragments [n = 32 kk + 8 l4 + e][d]
      u16x4_t lh4[MODE == kPair ? NBN : 1], ll4[MODE == kPair ? NBN : 1];   // kPair: [n = 16 nb + 4 l4 + e][d]
      if constexpr (MODE == kPair) {
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) rr::bf_split4(plm4[k][nb], lh4[nb], ll4[nb]);
      }
#pragma unroll
      for (int kk = 0; kk < NS / 32; ++kk) {
        if constexpr (MODE == kPair) {
        } else if constexpr (REG) {
          rr::bf_split8(plm[k][kk], lh8[kk], ll8[kk]);
        } else {
          lh8[kk] = frag(&m.LM_hi[16 * db + l15][32 * kk + 8 * l4]);
          ll8[kk] = frag(&m.LM_lo[16 * db + l15][32 * kk + 8 * l4]);
        }
      }
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        f32x4_t a1 = {0.f, 0.f, 0.f, 0.f}, a2 = {0.f, 0.f, 0.f, 0.f};
        {
          const int k0 = 8 * l4;
          const u16x8_t ph = frag(&m.y.PT_hi[16 * tb + l15][k0]), pl = frag(&m.y.PT_lo[16 * tb + l15][k0]);
          a1 = mfma16(ph, gh8, a1);
          a1 = mfma16(ph, gl8, a1);
          a1 = mfma16(pl, gh8, a1);
        }
        if constexpr (MODE == kPair) {
#pragma unroll
          for (int nb = 0; nb < NBN; ++nb) {
            const u16x4_t fa = frag4(&m.Kn[16 * tb + l15][16 * nb + 4 * l4]);
            a2 = mfma16k16(fa, lh4[nb], a2);
            a2 = mfma16k16(fa, ll4[nb], a2);
          }
        } else {
#pragma unroll
          for (int kk = 0; kk < NS / 32; ++kk) {
            const u16x8_t fa = frag(&m.Kn[16 * tb + l15][32 * kk + 8 * l4]);
            a2 = mfma16(fa, lh8[kk], a2);
            a2 = mfma16(fa, ll8[kk], a2);
          }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tb + 4 * l4 + r;
          rr::st_bf16_u32(duB, (uint32_t)(t * rsD + 16 * db + l15), m.w[t] * (a1[r] + m.m31[t] * a2[r]));
        }
      }
      if constexpr (MODE == kPair && CARRY) {
        // du's operand rows of the adjoint entering this chunk, for the
        // run's chunk before it: plm4 <- gam_31 plm4 + C^T diag(gam) dY (rows n,
        // columns d = this wave's du block; dY^T is the fragment above)
        const float g31 = m.gam[Q - 1];
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          const u16x8_t qf = rr::frag_tr(&m.Qn[0][16 * nb], ColBwdSmem<DH, NS, GLA, REG>::PN, lane);
          float qw[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) qw[e] = m.gam[8 * l4 + e] * bf_val(qf[e]);
          u16x8_t qh, ql;
          rr::bf_split8(qw, qh, ql);
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
          acc = mfma16(ql, gl8, acc);
          acc = mfma16(qh, gl8, acc);
          acc = mfma16(ql, gh8, acc);
          acc = mfma16(qh, gh8, acc);
          plm4[k][nb] = acc + g31 * plm4[k][nb];
        }
      }
    }
    float bz[2][4] = {};
    const float cd31 = m.cd[Q - 1], gam31 = m.gam[Q - 1];
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = w + 4 * cc;
      if (nb >= NBN) continue;
      float dAp = 0.f;
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        const int row = 16 * tb + l15, k0 = 8 * l4;
        f32x4_t ak = {0.f, 0.f, 0.f, 0.f}, aq = {0.f, 0.f, 0.f, 0.f}, akb = {0.f, 0.f, 0.f, 0.f};
        // B and C as B operands over s / t' (transposing reads of Kn / Qn)
        const u16x8_t fq = rr::frag_tr(&m.Qn[0][16 * nb], ColBwdSmem<DH, NS, GLA, REG>::PN, lane);
        ak = mfma16(frag(&m.y.MGT_hi[row][k0]), fq, ak);
        ak = mfma16(frag(&m.y.MGT_lo[row][k0]), fq, ak);
        const u16x8_t fk = rr::frag_tr(&m.Kn[0][16 * nb], ColBwdSmem<DH, NS, GLA, REG>::PN, lane);
        aq = mfma16(frag(&m.y.MG_hi[row][k0]), fk, aq);
        aq = mfma16(frag(&m.y.MG_lo[row][k0]), fk, aq);
        if constexpr (!GLA) {
          akb = mfma16(frag(&m.y.Km_hi[row][k0]), fk, akb);
          akb = mfma16(frag(&m.y.Km_lo[row][k0]), fk, akb);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tb + 4 * l4 + r, n = 16 * nb + l15;
          const uint32_t gi = (uint32_t)(t * rsN + n);
          const float z = ak[r] + m.m31[t] * ul[cc][tb][r];
          const float dbv = m.w[t] * z, dcv = m.gam[t] * gh[cc][tb][r] + aq[r];
          rr::st_bf16_u32(dBB, gi, dbv);
          rr::st_bf16_u32(dCB, gi, dcv);
          if constexpr (!GLA) {
            const float bv = bf_val(m.Kn[t][n]), cv = bf_val(m.Qn[t][n]);
            bz[tb][r] += bv * z;
            dAp += cv * (akb[r] + m.gam[t] * m.cd[t] * gh[cc][tb][r]) +
                   m.m31[t] * (cd31 - m.cd[t]) * m.w[t] * bv * ul[cc][tb][r];
          }
        }
      }
      if constexpr (!GLA) {
        dA_acc[cc] += rr::rows4_sum(dAp) + gam31 * cd31 * trn[cc];
      }
    }
    if constexpr (!GLA) {
      // sum_n B Z of this wave's columns
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = rr::row16_sum(bz[tb][r]);
          if (l15 == 0) m.BZp[w][16 * tb + 4 * l4 + r] = v;
        }
      }
    }
    if constexpr (carry) {
      // lam_prev = (gam o dY)^T C + gam_31 lam, blocks of this wave's columns
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        const int nb = w + 4 * cc;
        if (nb >= NBN) continue;
        const int k0 = 8 * l4;
        const u16x8_t qf = rr::frag_tr(&m.Qn[0][16 * nb], ColBwdSmem<DH, NS, GLA, REG>::PN, lane);
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
          for (int r = 0; r < 4; ++r) lam[cc][db][r] = acc[r] + gam31 * lam[cc][db][r];
        }
      }
    }
    if constexpr (!GLA) {
      __syncthreads();
      if (w == 0 && lane < Q) {
        const float bzt = m.BZp[0][lane] + m.BZp[1][lane] + m.BZp[2][lane] + m.BZp[3][lane];
        // T_t = R_t + sum_{t' >= t} gam X + sum_{s <= t} m31 w Y + m31_t gam_t tr
        const float tr = m.trw[0] + m.trw[1] + m.trw[2] + m.trw[3];
        const float T = (m.Rp[0][lane] + m.Rp[1][lane]) + (m.Rp[2][lane] + m.Rp[3][lane]) + m.Ts[0][lane] +
                        m.Ts[1][lane] + m.m31[lane] * m.gam[lane] * tr;
        rr::st_bf16(p.ddelta, baseX + lane * p.H, a * T + (1.f - a * m.xin[lane]) * bzt);
      }
    }
    if (MODE == kWhole || (MODE == kPair && CARRY)) __syncthreads();   // the next chunk rewrites the LDS
  };
  if constexpr (MODE == kPair) {
    chunk_body(cend - 1, std::true_type{}, std::true_type{});
    for (int c = cend - 2; c > cbeg; --c) chunk_body(c, std::false_type{}, std::true_type{});
    chunk_body(cbeg, std::false_type{}, std::false_type{});
  } else {
    for (int c = cend - 1; c >= cbeg; --c) chunk_body(c, std::false_type{}, std::false_type{});
  }
  if constexpr (!GLA) {
    // per-run dA partial of this lane's column
    const int nR = MODE == kWhole ? 1 : MODE == kPair ? p.nC / p.R : p.nC;
    const int run = MODE == kWhole ? 0 : MODE == kPair ? cbeg / p.R : cbeg;
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = w + 4 * cc;
      if (nb < NBN && l4 == 0) p.ws[rr::chunked::dA_slot(bh, nR, run) * NS + 16 * nb + l15] = dA_acc[cc];
    }
  }
  if (carry && p.dh0 != nullptr) {   // kWhole (kDirect stores dh0 in the direct sum)
#pragma unroll
    for (int cc = 0; cc < CPW; ++cc) {
      const int nb = w + 4 * cc;
      if (nb >= NBN) continue;
#pragma unroll
      for (int db = 0; db < NBD; ++db)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          p.dh0[bh * DH * NS + rr::chunked::state_off<GLA, DH, NS>(16 * db + 4 * l4 + r, 16 * nb + l15)] =
              lam[cc][db][r];
    }
  }
}

template <int DH, int NS, bool GLA>
int launch(const rr::ChunkArgs& p, int64_t B, hipStream_t s) {
  if (p.mode == kPipe) {
    if (int rc = rr::chunked::launch_scan<DH, NS, GLA>(p, B, s, true)) return rc;
    hipLaunchKernelGGL((col_bwd_kernel<DH, NS, kPipe, GLA>), rr::chunked::chunk_grid(p), dim3(256), 0, s, p);
  } else if (p.mode == rr::chunked::kPair) {
    if constexpr (GLA || DH > 64) {   // (the host picks it for SSD with Dh <= 64 only)
      return rr::fail(RR_EUNSUPPORTED, "chunked backward: no pair mode for this state");
    } else {
      if (p.R < 2 || p.nC % p.R != 0) return rr::fail(RR_EINVAL, "chunked backward: runs of R > 1 chunks dividing nC");
      if (int rc = rr::chunked::launch_scan<DH, NS, GLA>(p, B, s, true)) return rc;
      hipLaunchKernelGGL((col_bwd_kernel<DH, NS, rr::chunked::kPair, GLA>), rr::chunked::run_grid(p), dim3(256), 0, s,
                         p);
    }
  } else if (p.mode == kDirect) {
    // (wide: the states the host picks it for, SSD Dh 128 with N 64 and GLA Dh 128)
    if constexpr (!kWideDirect<DH, NS> || (DH % 64 == 0 && NS % 64 == 0 && (GLA || (DH == 128 && NS == 64))))
      hipLaunchKernelGGL((col_bwd_kernel<DH, NS, kDirect, GLA>), rr::chunked::chunk_grid(p), dim3(256), 0, s, p);
    else
      return rr::fail(RR_EUNSUPPORTED, "chunked backward: no direct mode for this state");
  } else {
    hipLaunchKernelGGL((col_bwd_kernel<DH, NS, kWhole, GLA>), dim3(1, p.H, (unsigned)B), dim3(256), 0, s, p);
  }
  return rr::check_launch("chunked backward");
}

}  // namespace

namespace rr {

int chunked_bwd_cols(const ChunkArgs& p, int64_t B, hipStream_t s, bool gla) {
  if (gla) {
    switch (p.DH) {
      case 32: return launch<32, 32, true>(p, B, s);
      case 64: return launch<64, 64, true>(p, B, s);
      case 128: return launch<128, 128, true>(p, B, s);
      default: return fail(RR_EUNSUPPORTED, "gla chunked backward: unsupported Dh");
    }
  }
  switch (p.DH * 1000 + p.NS) {
    case 32064: return launch<32, 64, false>(p, B, s);
    case 32128: return launch<32, 128, false>(p, B, s);
    case 64064: return launch<64, 64, false>(p, B, s);
    case 64128: return launch<64, 128, false>(p, B, s);
    case 128064: return launch<128, 64, false>(p, B, s);
    case 128128: return launch<128, 128, false>(p, B, s);
    default: return fail(RR_EUNSUPPORTED, "ssd chunked backward: unsupported (Dh, N)");
  }
}

}  // namespace rr
