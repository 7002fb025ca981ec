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
using rr::mfma16;
using rr::mfma32;
using rr::u16x8_t;
using rr::chunked::PQ;
using rr::chunked::Q;
using rr::chunked::r32row;

// LDS of the backward kernel.  The operands that die after phase B1 (x) share
// space with the masked products written in phase B2 (y).
template <int D>
struct GlaBwdSmem {
  static constexpr int PD = D + 8;
  uint16_t Kn[Q][PD];                    // k   [s][i]
  uint16_t Qn[Q][PD];                    // q   [t][i]
  uint16_t KT[D][PQ];                    // k^T [i][s]
  uint16_t QT[D][PQ];                    // q^T [i][t]
  uint16_t GYT_hi[D][PQ], GYT_lo[D][PQ]; // dY^T [j][t]
  uint16_t LM_hi[D][PD], LM_lo[D][PD];   // lam [j][i]
  float GH[Q][D + 1];                    // dY h_in [t][i]
  float UL[Q][D + 1];                    // V lam   [s][i]
  union {
    struct {                             // phase A -> B1
      uint16_t V[Q][PD];                     // v [s][j]
      uint16_t GY_hi[Q][PD], GY_lo[Q][PD];   // dY [t][j]
      uint16_t LMT_hi[D][PD], LMT_lo[D][PD]; // lam^T [i][j]
      uint16_t HT_hi[D][PD], HT_lo[D][PD];   // h_in^T [i][j]
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
  float XY[2][Q];                        // X, Y
  float g[Q], gam[Q], m31[Q];
  float trw[4];
};

template <int D>
__global__ __launch_bounds__(256) void gla_bwd_kernel(rr::ChunkArgs p) {
  constexpr int NBN = D / 16, NB = NBN * NBN, NBW = (NB + 3) / 4;
  __shared__ GlaBwdSmem<D> m;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int64_t rowH = p.H;
  const int64_t bh = (int64_t)b * p.H + h;
  const int64_t row0 = (int64_t)b * p.L + (int64_t)c * Q;  // first (b, t) row of the chunk

  // ------------------------------------------------ A: stage (all loads first)
  {
    constexpr int UV = (Q * D / 8 + 255) / 256, GV = (Q * D / 4 + 255) / 256;
    u16x8_t vv[UV], kv[UV], qv[UV];
    float4 gv[GV];
    f32x4_t lam[NBW], hin[NBW];
    float xv = 1.f;
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + 256 * v, tl = (i / (D / 8)) & (Q - 1), d0 = 8 * (i % (D / 8));
      const bool ok = i < Q * D / 8;
      const int64_t g = ((row0 + tl) * rowH + h) * D + d0;
      vv[v] = ok ? *reinterpret_cast<const u16x8_t*>(p.u + g) : u16x8_t{};
      kv[v] = ok ? *reinterpret_cast<const u16x8_t*>(p.Bm + g) : u16x8_t{};
      qv[v] = ok ? *reinterpret_cast<const u16x8_t*>(p.Cm + g) : u16x8_t{};
    }
#pragma unroll
    for (int v = 0; v < GV; ++v) {
      const int i = tid + 256 * v, tl = (i / (D / 4)) & (Q - 1), d0 = 4 * (i % (D / 4));
      gv[v] = i < Q * D / 4 ? *reinterpret_cast<const float4*>(p.dy + ((row0 + tl) * rowH + h) * D + d0)
                            : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (tid < Q) xv = bf_val(p.delta[(row0 + tid) * rowH + h]);
    const float* lsrc = p.agg + (bh * p.nC + c) * D * D;
    const float* hsrc = c > 0 ? p.ckpt + (bh * p.nC + c - 1) * D * D
                              : (p.h0 != nullptr ? p.h0 + bh * D * D : nullptr);
#pragma unroll
    for (int jj = 0; jj < NBW; ++jj) {
      const int j = w + 4 * jj;
      lam[jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      hin[jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      if (j < NB) {
        const int db = j / NBN, nb = j % NBN;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 16 * db + 4 * (lane >> 4) + r, n = 16 * nb + (lane & 15);
          lam[jj][r] = lsrc[d * D + n];
          if (hsrc != nullptr) hin[jj][r] = hsrc[c > 0 ? d * D + n : rr::chunked::state_off<true, D, D>(d, n)];
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
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint16_t hi, lo;
          bf_split(g4[e], hi, lo);
          m.x.GY_hi[tl][d0 + e] = hi;
          m.x.GY_lo[tl][d0 + e] = lo;
          m.GYT_hi[d0 + e][tl] = hi;
          m.GYT_lo[d0 + e][tl] = lo;
        }
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
    for (int jj = 0; jj < NBW; ++jj) {
      const int j = w + 4 * jj;
      if (j < NB) {
        const int db = j / NBN, nb = j % NBN;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int d = 16 * db + 4 * (lane >> 4) + r, n = 16 * nb + (lane & 15);
          uint16_t hi, lo;
          bf_split(lam[jj][r], hi, lo);
          m.LM_hi[d][n] = hi;
          m.LM_lo[d][n] = lo;
          m.x.LMT_hi[n][d] = hi;
          m.x.LMT_lo[n][d] = lo;
          bf_split(hin[jj][r], hi, lo);
          m.x.HT_hi[n][d] = hi;
          m.x.HT_lo[n][d] = lo;
          part += lam[jj][r] * hin[jj][r];
        }
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o);
    if (lane == 0) m.trw[w] = part;
  }
  __syncthreads();
  // ------------------------------------------------ B1: CB, G2 (32x32), GH, UL (32 x D)
  if (w == 0) {
    f32x16_t cb = {};
#pragma unroll
    for (int kb = 0; kb < D / 16; ++kb)
      cb = mfma32(frag(&m.Qn[lane & 31][16 * kb + 8 * (lane >> 5)]),
                  frag(&m.Kn[lane & 31][16 * kb + 8 * (lane >> 5)]), cb);
#pragma unroll
    for (int r = 0; r < 16; ++r) m.CB[r32row(r, lane)][lane & 31] = cb[r];
  } else if (w == 1) {
    f32x16_t g2 = {};
#pragma unroll
    for (int kb = 0; kb < D / 16; ++kb) {
      const u16x8_t fb = frag(&m.x.V[lane & 31][16 * kb + 8 * (lane >> 5)]);
      g2 = mfma32(frag(&m.x.GY_hi[lane & 31][16 * kb + 8 * (lane >> 5)]), fb, g2);
      g2 = mfma32(frag(&m.x.GY_lo[lane & 31][16 * kb + 8 * (lane >> 5)]), fb, g2);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) m.G2[r32row(r, lane)][lane & 31] = g2[r];
  } else {
    // GH blocks (tb, nb) then UL blocks (sb, nb), 16x16 each, on waves 2 and 3
    for (int task = w - 2; task < 4 * NBN; task += 2) {
      const bool isGH = task < 2 * NBN;
      const int tt = isGH ? task : task - 2 * NBN;
      const int tb = tt / NBN, nb = tt % NBN;
      const int row = 16 * tb + (lane & 15), col = 16 * nb + (lane & 15);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < D / 32; ++kb) {
        const int k0 = 32 * kb + 8 * (lane >> 4);
        if (isGH) {
          const u16x8_t ah = frag(&m.x.GY_hi[row][k0]), al = frag(&m.x.GY_lo[row][k0]);
          const u16x8_t bh = frag(&m.x.HT_hi[col][k0]), bl = frag(&m.x.HT_lo[col][k0]);
          acc = mfma16(ah, bh, acc);
          acc = mfma16(ah, bl, acc);
          acc = mfma16(al, bh, acc);
        } else {
          const u16x8_t fa = frag(&m.x.V[row][k0]);
          acc = mfma16(fa, frag(&m.x.LMT_hi[col][k0]), acc);
          acc = mfma16(fa, frag(&m.x.LMT_lo[col][k0]), acc);
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * tb + 4 * (lane >> 4) + r;
        if (isGH) m.GH[t][col] = acc[r];
        else m.UL[t][col] = acc[r];
      }
    }
  }
  __syncthreads();
  // ------------------------------------------------ B2: masked products; dg
  if (w != 2) {
    // wave 0: P^T; wave 1: MG^T; wave 3: MG
    float md[16];
    rr::chunked::decay_block32<true>(m.g, 0.f, lane, md);
    const int s = lane & 31;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int tp = r32row(r, lane);
      uint16_t hi, lo;
      if (w == 0) {
        bf_split(md[r] * m.CB[tp][s], hi, lo);
        m.y.PT_hi[s][tp] = hi;
        m.y.PT_lo[s][tp] = lo;
      } else {
        bf_split(md[r] * m.G2[tp][s], hi, lo);
        if (w == 1) {
          m.y.MGT_hi[s][tp] = hi;
          m.y.MGT_lo[s][tp] = lo;
        } else {
          m.y.MG_hi[tp][s] = hi;
          m.y.MG_lo[tp][s] = lo;
        }
      }
    }
  } else {
    {
      const int t = lane & 31;
      float acc = 0.f;
      if (lane < Q) {
#pragma unroll 8
        for (int n = 0; n < D; ++n) acc += m.GH[t][n] * bf_val(m.Qn[t][n]);
      } else {
#pragma unroll 8
        for (int n = 0; n < D; ++n) acc += m.UL[t][n] * bf_val(m.Kn[t][n]);
      }
      m.XY[lane >> 5][t] = acc;
    }
    rr::wave_lds_sync();
    if (lane <= Q) {
      const int row = lane;
      float e[Q], fv[Q];
      float f;
      if (row < Q) {
        f = m.XY[0][row];
#pragma unroll
        for (int s = 0; s < Q; ++s) e[s] = s < row ? m.CB[row][s] * m.G2[row][s] : 0.f;
      } else {
        f = m.trw[0] + m.trw[1] + m.trw[2] + m.trw[3];
#pragma unroll
        for (int s = 0; s < Q; ++s) e[s] = m.XY[1][s];
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
      rr::st_bf16(p.ddelta, (row0 + lane) * rowH + h, hp);
    }
  }
  __syncthreads();
  // ------------------------------------------------ C: dv, dk, dq
  if (w < D / 32) {
    const int d0 = 32 * w;
    f32x16_t a1 = {}, a2 = {};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int k0 = 16 * kb + 8 * (lane >> 5);
      const u16x8_t ph = frag(&m.y.PT_hi[lane & 31][k0]), pl = frag(&m.y.PT_lo[lane & 31][k0]);
      const u16x8_t gh = frag(&m.GYT_hi[d0 + (lane & 31)][k0]), gl = frag(&m.GYT_lo[d0 + (lane & 31)][k0]);
      a1 = mfma32(ph, gh, a1);
      a1 = mfma32(ph, gl, a1);
      a1 = mfma32(pl, gh, a1);
    }
#pragma unroll
    for (int kb = 0; kb < D / 16; ++kb) {
      const int k0 = 16 * kb + 8 * (lane >> 5);
      const u16x8_t fa = frag(&m.Kn[lane & 31][k0]);
      a2 = mfma32(fa, frag(&m.LM_hi[d0 + (lane & 31)][k0]), a2);
      a2 = mfma32(fa, frag(&m.LM_lo[d0 + (lane & 31)][k0]), a2);
    }
    const int d = d0 + (lane & 31);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = r32row(r, lane);
      rr::st_bf16(p.du, ((row0 + t) * rowH + h) * D + d, a1[r] + m.m31[t] * a2[r]);
    }
  } else {
    // dk (kind 0) and dq (kind 1) blocks over the waves >= D/32
    const int nw = 4 - D / 32;
    for (int task = w - D / 32; task < 4 * NBN; task += nw) {
      const int kind = task / (2 * NBN), tt = task % (2 * NBN);
      const int tb = tt / NBN, nb = tt % NBN;
      const int row = 16 * tb + (lane & 15), col = 16 * nb + (lane & 15);
      const int k0 = 8 * (lane >> 4);
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      if (kind == 0) {
        const u16x8_t fb = frag(&m.QT[col][k0]);
        acc = mfma16(frag(&m.y.MGT_hi[row][k0]), fb, acc);
        acc = mfma16(frag(&m.y.MGT_lo[row][k0]), fb, acc);
      } else {
        const u16x8_t fb = frag(&m.KT[col][k0]);
        acc = mfma16(frag(&m.y.MG_hi[row][k0]), fb, acc);
        acc = mfma16(frag(&m.y.MG_lo[row][k0]), fb, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * tb + 4 * (lane >> 4) + r;
        const int64_t gi = ((row0 + t) * rowH + h) * D + col;
        if (kind == 0) rr::st_bf16(p.dB, gi, acc[r] + m.m31[t] * m.UL[t][col]);
        else rr::st_bf16(p.dC, gi, m.gam[t] * m.GH[t][col] + acc[r]);
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
  hipLaunchKernelGGL((rr::chunked::agg_kernel<D, D, true>), dim3(p.nC, p.H, (unsigned)B), dim3(64), 0, s, p, 1);
  if (int rc = rr::check_launch("gla chunked backward aggregates")) return rc;
  hipLaunchKernelGGL((rr::chunked::pass_kernel<D, D, true>), dim3(D * D / 256, p.H, (unsigned)B), dim3(256), 0, s,
                     p, 1);
  if (int rc = rr::check_launch("gla chunked backward adjoint pass")) return rc;
  hipLaunchKernelGGL((gla_bwd_kernel<D>), dim3(p.nC, p.H, (unsigned)B), dim3(256), 0, s, p);
  return rr::check_launch("gla chunked backward");
}

int64_t align64(int64_t n) { return (n + 63) / 64 * 64; }

}  // namespace

namespace rr {

bool gla2_supported(int dtype, int64_t L, int64_t seg, int64_t Dh, int pass) {
  if (dtype != RR_BF16 || chunk_len(L, seg) != chunked::Q) return false;
  if (pass == 0) return Dh == 32 || Dh == 64 || Dh == 128;
  return Dh == 32 || Dh == 64;
}

size_t gla2_ws_bytes(int64_t B, int64_t H, int64_t nC, int64_t Dh, int pass) {
  int64_t f = align64(B * H * nC);
  if (pass == 1) f += align64(B * H * nC * Dh * Dh);
  return (size_t)f * sizeof(float);
}

void gla2_carve_ws(ChunkArgs& a, void* ws, int64_t B, int pass) {
  float* f = static_cast<float*>(ws);
  a.ws = nullptr;
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
