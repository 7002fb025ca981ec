// ssd_chunked.hip — SSD scan with a head-uniform decay rate on bf16 MFMA.
//
// When A_neg[h, n] is the same for every n (Mamba-2's per-head A, as in the
// benchmarked SSD configurations), the decay from step s to step t of a chunk is one scalar
// per head, M[t, s] = exp(a (cd_t - cd_s)) (cd = in-chunk cumulative delta), and
// a 32-step chunk of the recurrence (reference ssd.py:85-111) becomes dense
// products (the "SSD dual" form, rr_chunked.h).  The forward kernels are the
// shared ones of rr_chunked.h; this file holds the SSD backward.
//
// Work decomposition: a workgroup of 4 waves owns a run of R consecutive chunks
// of one (batch, head) and walks them in order, keeping the state h [Dh x N]
// (forward) or the adjoint (backward) in registers as 16x16 MFMA accumulator
// blocks, block j owned by wave j % 4.  The host picks R = all chunks of the
// head when there are enough heads to fill the GPU, else R = 1: then the
// chunk aggregates are formed first and one pass per state element carries
// the state (adjoint) across chunks (the pipelined mode of rr_chunked.h).
#include "rr_chunked.h"

#include <algorithm>

namespace {

using rr::bf_split;
using rr::bf_val;
using rr::f32x16_t;
using rr::f32x4_t;
using rr::frag;
using rr::mfma16;
using rr::mfma32;
using rr::u16x4_t;
using rr::u16x8_t;
using rr::chunked::Cfg;
using rr::chunked::prefix32;
using rr::chunked::PQ;
using rr::chunked::Q;
using rr::chunked::r32row;
using rr::chunked::kDirect;
using rr::chunked::kPipe;
using rr::chunked::kSum;
using rr::chunked::kWhole;
using rr::chunked::kRes;

}  // namespace

namespace rr {

bool ssd2_supported(int dtype, int64_t L, int64_t seg, int64_t Dh, int64_t N, int64_t A_stride_n) {
  if (dtype != RR_BF16 || A_stride_n != 0) return false;
  if (chunk_len(L, seg) != Q) return false;
  if (!(Dh == 32 || Dh == 64 || Dh == 128)) return false;
  if (!(N == 16 || N == 32 || N == 64 || N == 128)) return false;
  return true;
}

int ssd2_fwd(const ChunkArgs& p, int64_t B, hipStream_t s) {
  if (p.mode == kRes) return res_fwd(p, B, s, false);
  switch (p.DH * 1000 + p.NS) {
    case 32016: return chunked::launch_fwd<32, 16, false>(p, B, s);
    case 32032: return chunked::launch_fwd<32, 32, false>(p, B, s);
    case 32064: return chunked::launch_fwd<32, 64, false>(p, B, s);
    case 32128: return chunked::launch_fwd<32, 128, false>(p, B, s);
    case 64016: return chunked::launch_fwd<64, 16, false>(p, B, s);
    case 64032: return chunked::launch_fwd<64, 32, false>(p, B, s);
    case 64064: return chunked::launch_fwd<64, 64, false>(p, B, s);
    case 64128: return chunked::launch_fwd<64, 128, false>(p, B, s);
    case 128016: return chunked::launch_fwd<128, 16, false>(p, B, s);
    case 128032: return chunked::launch_fwd<128, 32, false>(p, B, s);
    case 128064: return chunked::launch_fwd<128, 64, false>(p, B, s);
    case 128128: return chunked::launch_fwd<128, 128, false>(p, B, s);
    default: return fail(RR_EUNSUPPORTED, "ssd chunked: unsupported (Dh, N)");
  }
}

}  // namespace rr

// ===================================================================== backward
//
// Per chunk (reference adjoint ssd.py:203-268 in matrix form), with lam the
// adjoint flowing in from later chunks (dL/dh_end through the next step),
// h_in the chunk's entering state (forward checkpoint), cd/gam/M as above and
// m31_t = M[31, t]:
//   CB = C B^T, G2 = dY U^T, P = M o CB, GH = dY h_in, UL = U lam
//   du = diag(delta) (P^T dY + diag(m31) B lam^T)
//   Z  = (M o G2)^T C + diag(m31) UL;   dB = diag(delta) Z
//   dC = diag(gam) GH + (M o G2 o delta_s) B
//   d(delta)_t = a T_t + (1 - a delta_t) sum_n B_t Z_t, where
//     T_t = sum_{d,n} lam_t h_t = R_t + sum_{t'>=t} gam X + sum_{s<=t} m31 delta Y + m31_t gam_t tr,
//     R_t = sum_{t'>=t} sum_{s<=t} (M o delta_s o G2 o CB)[t', s],
//     X = rowsum(GH o C), Y = rowsum(UL o B), tr = sum(lam o h_in)
//   dA[n] = sum_t' C (K B) + sum gam cd C GH + sum m31 delta (cd_31 - cd + delta) B UL
//           + gam_31 cd_31 sum_d lam h_in - sum delta^2 B Z,  K = M o delta_s o G2 o span
//   lam_prev = (gam o dY)^T C + gam_31 lam
// (derived from the per-step adjoint; checked against the float64 oracle).
// A whole-head run starts from lam = dfinal and carries lam_prev backwards in
// registers; a pipelined workgroup reads its lam from pass_kernel.

namespace {

// LDS of the backward kernel.  Arrays live in phase order, so the operands
// that die after phase B1 (x) share space with the masked products written in
// B2 (y).  The pipelined mode (CARRY false) takes dY^T, lam and the h_in / lam
// columns as register fragments straight from global memory instead of the
// transposed LDS copies (GYT, LM, LMT, HT), which keeps its LDS small enough
// for four workgroups per CU (N = 16; three with the sum mode's LS).  Arrays a
// mode does not use have no rows.
template <int DH, int NS, bool CARRY, bool SUM>
struct BwdSmem {
  static constexpr int PD = DH + 8, PN = NS + 8;
  static constexpr int TD = CARRY ? DH : 0, TN = CARRY ? NS : 0;
  float LS[SUM ? DH : 0][NS + 4];  // kSum: the summed lam [d][n], read back as register fragments
  uint16_t Bn[Q][PN];
  uint16_t Cn[Q][PN];
  uint16_t BT[NS][PQ];
  uint16_t CT[NS][PQ];
  uint16_t GYT_hi[TD][PQ], GYT_lo[TD][PQ];
  uint16_t LM_hi[TD][PN], LM_lo[TD][PN];
  float GH[Q][NS + 1];
  float UL[Q][NS + 1];
  union {
    struct {                       // phase A -> B1
      uint16_t U[Q][PD];
      uint16_t GY_hi[Q][PD], GY_lo[Q][PD];
      uint16_t LMT_hi[TN][PD], LMT_lo[TN][PD];
      uint16_t HT_hi[TN][PD], HT_lo[TN][PD];
    } x;
    struct {                       // phase B2 -> C
      uint16_t PT_hi[Q][PQ], PT_lo[Q][PQ];
      uint16_t MGT_hi[Q][PQ], MGT_lo[Q][PQ];
      uint16_t MGd_hi[Q][PQ], MGd_lo[Q][PQ];
      uint16_t Km_hi[Q][PQ], Km_lo[Q][PQ];
    } y;
  };
  float CB[Q][Q];                  // phase B1 -> B2 (rows read whole: unpadded)
  float G2[Q][Q];
  // (gam o C)^T, for the adjoint carried to the previous chunk (whole-head
  // mode; chunk 0 of the direct mode for the initial-state gradient)
  uint16_t CgT_hi[CARRY ? NS : 0][PQ], CgT_lo[CARRY ? NS : 0][PQ];
  float del[Q], cd[Q], gam[Q], m31[Q];
  float Rp[4][Q];                  // per-wave partials of R_t (phase B2)
  float Xs[NS / 16][Q], Ys[NS / 16][Q], BZs[NS / 16][Q];   // row sums over one 16-column block
  float Ts[2][Q];                  // suffix of gam X, prefix of m31 delta Y
  float t4[4][NS];
  float dAq[2][2][NS];             // dA partials of the (kind, tb) tasks
};

template <int DH, int NS, int MODE>
union BwdShared {
  BwdSmem<DH, NS, MODE != kPipe && MODE != kSum, MODE == kSum> m;
};
template <int DH, int NS>
union BwdShared<DH, NS, kSum> {
  BwdSmem<DH, NS, false, true> m;
  rr::chunked::DirectSmem<DH, NS, true> d;   // the adjoint's sum, before the chunk's staging
};

// One chunk per workgroup with lam from the workspace (kPipe, pass_kernel) or
// summed over the later chunks' inputs in the kernel (kSum, direct_sum); or a
// whole head per workgroup, lam carried backwards in registers (kWhole).
// Workgroups per CU: the pipelined mode as many as its LDS allows (up to 4),
// the sum mode 3, the whole-head mode 2.
template <int DH, int NS, int MODE>
constexpr int kBwdWgs = MODE == kPipe  ? (160 * 1024 / sizeof(BwdShared<DH, NS, MODE>) >= 4 ? 4 : 3)
                        : MODE == kSum ? 3
                                       : 2;

template <int DH, int NS, int MODE>
__global__ __launch_bounds__(256, (kBwdWgs<DH, NS, MODE>)) void ssd2_bwd_kernel(rr::ChunkArgs p) {
  using K = Cfg<DH, NS>;
  // PIPE: one chunk per workgroup with lam from the workspace (kPipe) or summed
  // in the kernel (kSum, SUM); the operands of du and of GH / UL are register
  // fragments
  constexpr bool SUM = MODE == kSum;
  constexpr bool PIPE = MODE == kPipe || SUM;
  __shared__ BwdShared<DH, NS, MODE> smu;
  auto& m = smu.m;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  int h, b, cbeg;
  if constexpr (MODE == kWhole) {
    h = blockIdx.y, b = blockIdx.z, cbeg = 0;
  } else {
    // early chunks cost most where the adjoint is a sum over the later ones
    const rr::chunked::ChunkId id = rr::chunked::chunk_id(p, MODE == kSum, false);
    if (!id.valid) return;
    h = id.h, b = id.b, cbeg = id.c;
  }
  // one chunk per workgroup except in the whole-head mode (a visible single
  // iteration keeps the compiler from hoisting addresses out of the loop)
  const int cend = MODE == kWhole ? min(cbeg + p.R, p.nC) : cbeg + 1;
  const float a = p.A[(int64_t)h * p.A_stride_h];
  const int64_t rowH = p.H;
  const int64_t sbase = ((int64_t)b * p.H + h) * DH * NS;
  constexpr int NBN = K::NBN;
  constexpr int NBD = DH / 16;   // du column blocks (phase C: one per wave w < NBD)
  static_assert(NBD == 2 || NBD == 4, "the du blocks map onto the four waves");

  f32x4_t lam[K::NBW];
#pragma unroll
  for (int jj = 0; jj < K::NBW; ++jj) lam[jj] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // the adjoint entering chunk c - 1 is needed for the whole head
  const bool carry = MODE == kWhole;
  const float* lsrc = MODE == kPipe ? p.agg + rr::chunked::adj_slot((int64_t)b * p.H + h, p.nC, 1, cbeg) * DH * NS
                                    : (p.dfinal != nullptr ? p.dfinal + sbase : nullptr);
  if (!SUM && lsrc != nullptr) {
#pragma unroll
    for (int jj = 0; jj < K::NBW; ++jj) {
      const int j = w + 4 * jj;
      if (j < K::NB) {
        const int db = j / NBN, nb = j % NBN;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          lam[jj][r] = lsrc[(16 * db + 4 * (lane >> 4) + r) * NS + 16 * nb + (lane & 15)];
      }
    }
  }
  float dA_acc = 0.f;  // thread tid < NS accumulates dA[h, tid] over the run

  for (int c = cend - 1; c >= cbeg; --c) {
    // a fresh copy of the thread index per chunk keeps the compiler from
    // hoisting every per-lane address of the body out of the chunk loop
    int tidv = tid;
    if constexpr (MODE == kWhole) asm volatile("" : "+v"(tidv));
    const int tid = tidv, lane = tidv & 63;
    const int64_t row0 = (int64_t)b * p.L + (int64_t)c * Q;
    // uniform chunk bases ([.., H, DH] and [.., H, NS] rows of step 0) and
    // 32-bit per-lane offsets (no 64-bit address math per element)
    const int64_t baseD = (row0 * rowH + h) * DH, baseN = (row0 * rowH + h) * NS;
    const uint32_t rsD = (uint32_t)(rowH * DH), rsN = (uint32_t)(rowH * NS);
    // ------------------------------------------------ A: stage (all loads first)
    f32x4_t hin[K::NBW];
    // pipelined mode: register operand fragments (see BwdSmem)
    constexpr int TPW = NBN;   // GH / UL tasks per task wave (waves 2 and 3 in phase B1)
    float pdy[PIPE ? 8 : 1], plm[PIPE ? NS / 16 : 1][4];
    f32x4_t pcol[PIPE ? TPW : 1][PIPE ? DH / 16 : 1];
    {
      constexpr int UV = (Q * DH / 8 + 255) / 256, BV = (Q * NS / 8 + 255) / 256, GV = (Q * DH / 4 + 255) / 256;
      u16x8_t uv[UV], bv[BV], cv[BV];
      float4 gv[GV];
      float dv = 0.f;
      // Every load below is issued by every thread, unconditionally and in
      // bounds (clamped indices; surplus values are multiplied by 0, which
      // the compiler cannot turn into a branch around the load): a load
      // under a branch makes the branch's join wait for all of them.
      auto issue = [&]() {
#pragma unroll
        for (int v = 0; v < UV; ++v) {
          const int i = tid + 256 * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
          uv[v] = rr::ld32<u16x8_t>(p.u + baseD, tl * rsD + d0);
        }
#pragma unroll
        for (int v = 0; v < BV; ++v) {
          const int i = tid + 256 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
          bv[v] = rr::ld32<u16x8_t>(p.Bm + baseN, tl * rsN + n0);
          cv[v] = rr::ld32<u16x8_t>(p.Cm + baseN, tl * rsN + n0);
        }
#pragma unroll
        for (int v = 0; v < GV; ++v) {
          const int i = tid + 256 * v, tl = (i / (DH / 4)) & (Q - 1), d0 = 4 * (i % (DH / 4));
          gv[v] = rr::ld32<float4>(p.dy + baseD, tl * rsD + d0);
        }
        dv = bf_val(p.delta[(row0 + (lane & (Q - 1))) * rowH + h]);   // lanes >= 32 masked at use
        // the entering state (checkpoint slot c - 1, or h0; none: zero, read
        // from the checkpoint buffer and dropped)
        const float has_h = c > 0 || p.h0 != nullptr ? 1.f : 0.f;   // the slot read is finite
        const auto hsrc = rr::as_global(c > 0 ? p.ckpt + (((int64_t)b * p.H + h) * p.nC + (c - 1)) * DH * NS
                                              : (p.h0 != nullptr ? p.h0 + sbase : p.ckpt));
        if constexpr (PIPE) {
          // GH / UL tasks of waves 2 and 3: the h_in / lam column nb as
          // 16x16x16 B fragments (k = d); waves 0 and 1 load and drop them
#pragma unroll
          for (int q = 0; q < TPW; ++q) {
            const int task = (w & 1) + 2 * q;
            const int kind = task / NBN, nb = task % NBN;
            // lam (kind 1) comes from LDS after the staging barrier in the sum mode
            const float use = task < 2 * NBN ? (kind == 0 ? has_h : SUM ? 0.f : 1.f) : 0.f;
            const auto src = kind == 0 || SUM ? hsrc : rr::as_global(lsrc);
#pragma unroll
            for (int kb = 0; kb < DH / 16; ++kb)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float v = src[(16 * kb + 4 * (lane >> 4) + e) * NS + 16 * (nb & (NBN - 1)) + (lane & 15)];
                pcol[q][kb][e] = use * v;
              }
          }
        }
#pragma unroll
        for (int jj = 0; jj < K::NBW; ++jj) {
          const int j = w + 4 * jj;
          const int jc = min(j, K::NB - 1), db = jc / NBN, nb = jc % NBN;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float v = hsrc[(16 * db + 4 * (lane >> 4) + r) * NS + 16 * nb + (lane & 15)];
            hin[jj][r] = (j < K::NB ? has_h : 0.f) * v;
          }
        }
      };
      if constexpr (SUM) {
        // lam summed over the later chunks' inputs; the chunk's own loads go
        // out when each wave has staged its last summed chunk; the chunk-0
        // workgroup also writes dh0
        // (DH = 64, NS = 16: wave w's block j = w comes back summed in `own`)
        constexpr bool OWN = DH == 64 && NS == 16;
        f32x4_t own[1];
        const float gam_all =
            rr::chunked::direct_sum<DH, NS, false, true, true>(p, cbeg, b, h, a, smu.d, p.dh0, issue, own);
        const float* dfb = p.dfinal != nullptr ? p.dfinal + sbase : nullptr;
        if constexpr (OWN) {
          lam[0] = own[0];
        } else {
#pragma unroll
          for (int jj = 0; jj < K::NBW; ++jj) {
            const int j = w + 4 * jj;
            if (j < K::NB) {
              const int db = j / NBN, nb = j % NBN;
#pragma unroll
              for (int r = 0; r < 4; ++r)
                lam[jj][r] = rr::chunked::direct_partial(smu.d, 16 * db + 4 * (lane >> 4) + r, 16 * nb + (lane & 15));
            }
          }
        }
        if (dfb != nullptr) {
#pragma unroll
          for (int jj = 0; jj < K::NBW; ++jj) {
            const int j = w + 4 * jj;
            if (j < K::NB) {
              const int db = j / NBN, nb = j % NBN;
#pragma unroll
              for (int r = 0; r < 4; ++r)
                lam[jj][r] += rr::chunked::direct_ext<DH, NS, false>(gam_all, dfb, 16 * db + 4 * (lane >> 4) + r,
                                                                     16 * nb + (lane & 15));
            }
          }
        }
        __syncthreads();   // the sum's LDS is dead: the staging below reuses it
        // the summed lam for the register fragments (read after the staging barrier)
#pragma unroll
        for (int jj = 0; jj < K::NBW; ++jj) {
          const int j = w + 4 * jj;
          if (j < K::NB) {
            const int db = j / NBN, nb = j % NBN;
#pragma unroll
            for (int r = 0; r < 4; ++r) m.LS[16 * db + 4 * (lane >> 4) + r][16 * nb + (lane & 15)] = lam[jj][r];
          }
        }
      } else {
        issue();
      }
      // LDS writes
#pragma unroll
      for (int v = 0; v < UV; ++v) {
        const int i = tid + 256 * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
        if (i < Q * DH / 8) *reinterpret_cast<u16x8_t*>(&m.x.U[tl][d0]) = uv[v];
      }
#pragma unroll
      for (int v = 0; v < BV; ++v) {
        const int i = tid + 256 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
        if (i < Q * NS / 8) {
          *reinterpret_cast<u16x8_t*>(&m.Bn[tl][n0]) = bv[v];
          *reinterpret_cast<u16x8_t*>(&m.Cn[tl][n0]) = cv[v];
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            m.BT[n0 + e][tl] = bv[v][e];
            m.CT[n0 + e][tl] = cv[v][e];
          }
        }
      }
#pragma unroll
      for (int v = 0; v < GV; ++v) {
        const int i = tid + 256 * v, tl = (i / (DH / 4)) & (Q - 1), d0 = 4 * (i % (DH / 4));
        if (i < Q * DH / 4) {
          const float g4[4] = {gv[v].x, gv[v].y, gv[v].z, gv[v].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            uint16_t hi, lo;
            bf_split(g4[e], hi, lo);
            m.x.GY_hi[tl][d0 + e] = hi;
            m.x.GY_lo[tl][d0 + e] = lo;
            if constexpr (!PIPE) {
              m.GYT_hi[d0 + e][tl] = hi;
              m.GYT_lo[d0 + e][tl] = lo;
            }
          }
        }
      }
      if (w == 0) {
        const float cdv = prefix32(lane < Q ? dv : 0.f, lane);
        const float c31 = __shfl(cdv, 31);
        if (lane < Q) {
          const float gt = __expf(a * cdv), mt = __expf(a * (c31 - cdv));
          m.del[lane] = dv;
          m.cd[lane] = cdv;
          m.gam[lane] = gt;
          m.m31[lane] = mt;
        }
      }
#pragma unroll
      for (int jj = 0; jj < K::NBW; ++jj) {
        const int j = w + 4 * jj;
        if (!PIPE && j < K::NB) {
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
          }
        }
      }
    }
    __syncthreads();
    // ------------------------------------------------ B1: CB, G2 (32x32), GH, UL (16x16), (gam o C)^T
    if (w == 0) {
      f32x16_t cb = {};
#pragma unroll
      for (int kb = 0; kb < NS / 16; ++kb)
        cb = mfma32(frag(&m.Cn[lane & 31][16 * kb + 8 * (lane >> 5)]),
                    frag(&m.Bn[lane & 31][16 * kb + 8 * (lane >> 5)]), cb);
#pragma unroll
      for (int r = 0; r < 16; ++r) m.CB[r32row(r, lane)][lane & 31] = cb[r];
    } else if (w == 1) {
      f32x16_t g2 = {};
#pragma unroll
      for (int kb = 0; kb < DH / 16; ++kb) {
        const u16x8_t fb = frag(&m.x.U[lane & 31][16 * kb + 8 * (lane >> 5)]);
        g2 = mfma32(frag(&m.x.GY_hi[lane & 31][16 * kb + 8 * (lane >> 5)]), fb, g2);
        g2 = mfma32(frag(&m.x.GY_lo[lane & 31][16 * kb + 8 * (lane >> 5)]), fb, g2);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) m.G2[r32row(r, lane)][lane & 31] = g2[r];
    } else if constexpr (PIPE) {
      // tasks (kind, nb): GH = dY h_in (kind 0) or UL = U lam (kind 1) for the
      // 16 columns nb, B fragments from registers
      const int l15 = lane & 15, l4 = lane >> 4;
#pragma unroll
      for (int q = 0; q < TPW; ++q) {
        const int task = (w - 2) + 2 * q;
        const int kind = task / NBN, nb = task % NBN;
        if (SUM && kind == 1) {
#pragma unroll
          for (int kb = 0; kb < DH / 16; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e) pcol[q][kb][e] = m.LS[16 * kb + 4 * l4 + e][16 * nb + l15];
        }
        u16x4_t bh[DH / 16], bl[DH / 16];
#pragma unroll
        for (int kb = 0; kb < DH / 16; ++kb) rr::bf_split4(pcol[q][kb], bh[kb], bl[kb]);
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          const int row = 16 * tb + l15;
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < DH / 16; ++kb) {
            const int k0 = 16 * kb + 4 * l4;
            if (kind == 0) {
              const u16x4_t ah = rr::frag4(&m.x.GY_hi[row][k0]), al = rr::frag4(&m.x.GY_lo[row][k0]);
              acc = rr::mfma16k16(ah, bh[kb], acc);
              acc = rr::mfma16k16(ah, bl[kb], acc);
              acc = rr::mfma16k16(al, bh[kb], acc);
            } else {
              const u16x4_t av = rr::frag4(&m.x.U[row][k0]);
              acc = rr::mfma16k16(av, bh[kb], acc);
              acc = rr::mfma16k16(av, bl[kb], acc);
            }
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * tb + 4 * l4 + r, col = 16 * nb + l15;
            if (kind == 0) m.GH[t][col] = acc[r];
            else m.UL[t][col] = acc[r];
          }
        }
      }
    } else {
      // tasks: GH blocks (tb, nb) and UL blocks (sb, nb); waves 2 and 3
      for (int task = w - 2; task < 4 * NBN; task += 2) {
        const bool isGH = task < 2 * NBN;
        const int tt = isGH ? task : task - 2 * NBN;
        const int tb = tt / NBN, nb = tt % NBN;
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
        const int row = 16 * tb + (lane & 15), col = 16 * nb + (lane & 15);
#pragma unroll
        for (int kb = 0; kb < DH / 32; ++kb) {
          const int k0 = 32 * kb + 8 * (lane >> 4);
          if (isGH) {
            const u16x8_t ah = frag(&m.x.GY_hi[row][k0]), al = frag(&m.x.GY_lo[row][k0]);
            const u16x8_t bh = frag(&m.x.HT_hi[col][k0]), bl = frag(&m.x.HT_lo[col][k0]);
            acc = mfma16(ah, bh, acc);
            acc = mfma16(ah, bl, acc);
            acc = mfma16(al, bh, acc);
          } else {
            const u16x8_t fa = frag(&m.x.U[row][k0]);
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
      if constexpr (MODE != kPipe) {
        if (carry) {
          for (int i = tid - 128; i < NS * Q; i += 128) {
            const int n = i / Q, t = i % Q;
            uint16_t hi, lo;
            bf_split(m.gam[t] * bf_val(m.Cn[t][n]), hi, lo);
            m.CgT_hi[n][t] = hi;
            m.CgT_lo[n][t] = lo;
          }
        }
      }
    }
    __syncthreads();
    // ------------------------------------------------ B2: masked products, rectangle sums
    if constexpr (PIPE) {
      // du operands (used in phase C by waves w < NBD; the loads land while
      // B2 runs): the 16x16 B fragments of du's column block d = 16 w + l15,
      // dY^T [t' = 8 l4 + e][d] and lam^T [n = 16 kk + 4 l4 + e][d].  Every
      // wave issues them (waves without a du block repeat one), so no branch
      // join waits for the loads.
      const int d = 16 * (w & (NBD - 1)) + (lane & 15), l4 = lane >> 4;
#pragma unroll
      for (int e = 0; e < 8; ++e) pdy[e] = rr::ld32<float>(p.dy + baseD, (8 * l4 + e) * rsD + d);
#pragma unroll
      for (int kk = 0; kk < NS / 16; ++kk) {
        const float* src = SUM ? &m.LS[d][16 * kk + 4 * l4] : lsrc + d * NS + 16 * kk + 4 * l4;
        const float4 l0 = *reinterpret_cast<const float4*>(src);
        plm[kk][0] = l0.x, plm[kk][1] = l0.y, plm[kk][2] = l0.z, plm[kk][3] = l0.w;
      }
    }
    {
      // Wave w forms rows t' = t0 + q, q < 4, t0 = 8 w + 4 (lane / 32), of
      // every 32 x 32 product, column s = lane % 32 (one decay per element):
      //   P^T = (M o CB)^T and (M o G2)^T, [s][t'] (four consecutive t': one
      //   8-byte write each); M o G2 o delta_s and K = M o G2 o delta_s o
      //   (cd_t' - cd_s + delta_s), [t'][s];
      //   R_t = sum_{t' >= t} sum_{s <= t} E[t', s], E = M o delta_s o G2 o CB:
      //   a prefix over s along the lanes, the rows t' >= s of column s, and
      //   this wave's partial over its rows (summed in phase D).
      const int s = lane & 31, t0 = 8 * w + 4 * (lane >> 5);
      const float cds = m.cd[s], ds = m.del[s];
      float pt[4], mg[4], rs = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int tp = t0 + q;
        const float ctp = m.cd[tp];
        const float md = rr::chunked::masked_exp(s <= tp, a * (ctp - cds));
        const float cb = m.CB[tp][s];
        pt[q] = md * cb;
        mg[q] = md * m.G2[tp][s];
        const float mgd = mg[q] * ds;
        uint16_t hi, lo;
        bf_split(mgd, hi, lo);
        m.y.MGd_hi[tp][s] = hi;
        m.y.MGd_lo[tp][s] = lo;
        bf_split(mgd * (ctp - cds + ds), hi, lo);
        m.y.Km_hi[tp][s] = hi;
        m.y.Km_lo[tp][s] = lo;
        const float k = rr::prefix32_sum(mgd * cb);
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
    }
    __syncthreads();
    // ------------------------------------------------ C: du, Z/dB, dC, KB, lam_prev
    const float gam31 = m.gam[Q - 1];
    {
      const int l15 = lane & 15, l4 = lane >> 4;
      if (w < NBD) {
        // du, column block d = 16 w + l15:
        // du = diag(delta) (P^T dY + diag(m31) B lam^T)
        const int d = 16 * w + l15;
        u16x8_t gh, gl;   // dY^T [t' = 8 l4 + e][d]
        if constexpr (PIPE) {
          rr::bf_split8(pdy, gh, gl);
        } else {
          gh = frag(&m.GYT_hi[d][8 * l4]);
          gl = frag(&m.GYT_lo[d][8 * l4]);
        }
        u16x4_t lh[NS / 16], ll[NS / 16];   // lam^T [n = 16 kk + 4 l4 + e][d]
#pragma unroll
        for (int kk = 0; kk < NS / 16; ++kk) {
          if constexpr (PIPE) {
            rr::bf_split4(f32x4_t{plm[kk][0], plm[kk][1], plm[kk][2], plm[kk][3]}, lh[kk], ll[kk]);
          } else {
            lh[kk] = rr::frag4(&m.LM_hi[d][16 * kk + 4 * l4]);
            ll[kk] = rr::frag4(&m.LM_lo[d][16 * kk + 4 * l4]);
          }
        }
#pragma unroll
        for (int tb = 0; tb < 2; ++tb) {
          f32x4_t a1 = {0.f, 0.f, 0.f, 0.f}, a2 = {0.f, 0.f, 0.f, 0.f};
          const u16x8_t ph = frag(&m.y.PT_hi[16 * tb + l15][8 * l4]), pl = frag(&m.y.PT_lo[16 * tb + l15][8 * l4]);
          a1 = mfma16(ph, gh, a1);
          a1 = mfma16(ph, gl, a1);
          a1 = mfma16(pl, gh, a1);
#pragma unroll
          for (int kk = 0; kk < NS / 16; ++kk) {
            const u16x4_t fb = rr::frag4(&m.Bn[16 * tb + l15][16 * kk + 4 * l4]);
            a2 = rr::mfma16k16(fb, lh[kk], a2);
            a2 = rr::mfma16k16(fb, ll[kk], a2);
          }
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 16 * tb + 4 * l4 + r;
            rr::st_bf16_u32(p.du + baseD, t * rsD + d, m.del[t] * (a1[r] + m.m31[t] * a2[r]));
          }
        }
      }
      // Z / dB and dC (+ K B) blocks, spread over the four waves, with their
      // row sums (sum_n B Z, Y = sum_n UL B, X = sum_n GH C) and dA partials
      const float cd31 = m.cd[Q - 1];
      for (int task = w; task < 4 * NBN; task += 4) {
        const int kind = task / (2 * NBN), tt = task % (2 * NBN);
        const int tb = tt / NBN, nb = tt % NBN;
        const int row = 16 * tb + (lane & 15), col = 16 * nb + (lane & 15);
        const int k0 = 8 * (lane >> 4);
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f}, akb = {0.f, 0.f, 0.f, 0.f};
        if (kind == 0) {
          const u16x8_t fb = frag(&m.CT[col][k0]);
          acc = mfma16(frag(&m.y.MGT_hi[row][k0]), fb, acc);
          acc = mfma16(frag(&m.y.MGT_lo[row][k0]), fb, acc);
        } else {
          const u16x8_t fb = frag(&m.BT[col][k0]);
          acc = mfma16(frag(&m.y.MGd_hi[row][k0]), fb, acc);
          acc = mfma16(frag(&m.y.MGd_lo[row][k0]), fb, acc);
          akb = mfma16(frag(&m.y.Km_hi[row][k0]), fb, akb);
          akb = mfma16(frag(&m.y.Km_lo[row][k0]), fb, akb);
        }
        float da = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tb + 4 * (lane >> 4) + r;
          const uint32_t gi = t * rsN + col;
          float s1, s2;
          if (kind == 0) {
            const float bv = bf_val(m.Bn[t][col]), ul = m.UL[t][col], dt = m.del[t];
            const float z = acc[r] + m.m31[t] * ul;
            rr::st_bf16_u32(p.dB + baseN, gi, dt * z);
            s1 = bv * z;
            s2 = ul * bv;
            da += bv * (m.m31[t] * dt * (cd31 - m.cd[t] + dt) * ul - dt * dt * z);
          } else {
            const float cv = bf_val(m.Cn[t][col]), gh = m.GH[t][col];
            const float dc = m.gam[t] * gh + acc[r];
            rr::st_bf16_u32(p.dC + baseN, gi, dc);
            s1 = gh * cv;
            s2 = 0.f;
            da += cv * (akb[r] + m.gam[t] * m.cd[t] * gh);
          }
          s1 = rr::row16_sum(s1);
          s2 = rr::row16_sum(s2);
          if ((lane & 15) == 0) {
            if (kind == 0) {
              m.BZs[nb][t] = s1;
              m.Ys[nb][t] = s2;
            } else {
              m.Xs[nb][t] = s1;
            }
          }
        }
        da = rr::rows4_sum(da);
        if (lane < 16) m.dAq[kind][tb][col] = da;
      }
    }
    // lam_prev = (gam o dY)^T C + gam31 lam; sum_d lam h_in per n (for tr and dA)
    {
      float t4p[NBN];
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) t4p[nb] = 0.f;
#pragma unroll
      for (int jj = 0; jj < K::NBW; ++jj) {
        const int j = w + 4 * jj;
        if (j < K::NB) {
          const int db = j / NBN, nb = j % NBN;
          float part = 0.f;
#pragma unroll
          for (int r = 0; r < 4; ++r) part += lam[jj][r] * hin[jj][r];
          if constexpr (MODE != kPipe) if (carry) {
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
            const int k0 = 8 * (lane >> 4);
            const u16x8_t ah = frag(&m.GYT_hi[16 * db + (lane & 15)][k0]);
            const u16x8_t al = frag(&m.GYT_lo[16 * db + (lane & 15)][k0]);
            const u16x8_t bh = frag(&m.CgT_hi[16 * nb + (lane & 15)][k0]);
            const u16x8_t bl = frag(&m.CgT_lo[16 * nb + (lane & 15)][k0]);
            acc = mfma16(ah, bh, acc);
            acc = mfma16(ah, bl, acc);
            acc = mfma16(al, bh, acc);
#pragma unroll
            for (int r = 0; r < 4; ++r) lam[jj][r] = acc[r] + gam31 * lam[jj][r];
          }
          part += __shfl_xor(part, 16);
          part += __shfl_xor(part, 32);
#pragma unroll
          for (int q = 0; q < NBN; ++q)
            if (q == nb) t4p[q] += part;
        }
      }
      if (lane < 16) {
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) m.t4[w][16 * nb + lane] = t4p[nb];
      }
    }
    __syncthreads();
    // ------------------------------------------------ D: d(delta), dA
    // d(delta)_t = a T_t + (1 - a delta_t) sum_n B_t Z_t,
    // T_t = sum lam_t h_t = R_t + sum_{t' >= t} gam X + sum_{s <= t} m31 delta Y + m31_t gam_t tr
    if (w == 0) {
      const int ln = lane & (NS - 1);   // every lane reads, lanes >= NS drop it (no branch)
      const float tn = lane < NS ? m.t4[0][ln] + m.t4[1][ln] + m.t4[2][ln] + m.t4[3][ln] : 0.f;
      const float tr = rr::wave_sum(tn);
      // lanes 0..31: suffix of gam X in reversed lane order; lanes 32..63: prefix of m31 delta Y
      const int tq = lane < Q ? Q - 1 - lane : lane - Q;
      float xy = 0.f;
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) {
        const float xs = m.Xs[nb][tq], ys = m.Ys[nb][tq];   // both read, then selected (no branch)
        xy += lane < Q ? xs : ys;
      }
      const float gq = m.gam[tq], md = m.m31[tq] * m.del[tq];
      xy *= lane < Q ? gq : md;
      m.Ts[lane < Q ? 0 : 1][tq] = rr::prefix32_sum(xy);
      rr::wave_lds_sync();
      if (lane < Q) {
        const int t = lane;
        float bz = 0.f;
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) bz += m.BZs[nb][t];
        const float T = (m.Rp[0][t] + m.Rp[1][t]) + (m.Rp[2][t] + m.Rp[3][t]) + m.Ts[0][t] + m.Ts[1][t] +
                        m.m31[t] * m.gam[t] * tr;
        rr::st_bf16(p.ddelta, (row0 + t) * rowH + h, a * T + (1.f - a * m.del[t]) * bz);
      }
    } else if (w == 1 && lane < NS) {
      dA_acc += m.dAq[0][0][lane] + m.dAq[0][1][lane] + m.dAq[1][0][lane] + m.dAq[1][1][lane] +
                gam31 * m.cd[Q - 1] * (m.t4[0][lane] + m.t4[1][lane] + m.t4[2][lane] + m.t4[3][lane]);
    }
    if constexpr (MODE == kWhole) __syncthreads();   // the next chunk rewrites the LDS
  }
  // per-run dA partial and the initial-state gradient
  const int nR = MODE == kWhole ? 1 : p.nC;   // runs per head
  const int run = MODE == kWhole ? 0 : cbeg;
  if (w == 1 && lane < NS) p.ws[rr::chunked::dA_slot((int64_t)b * p.H + h, nR, run) * NS + lane] = dA_acc;
  if (carry && p.dh0 != nullptr) {
#pragma unroll
    for (int jj = 0; jj < K::NBW; ++jj) {
      const int j = w + 4 * jj;
      if (j < K::NB) {
        const int db = j / NBN, nb = j % NBN;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          p.dh0[sbase + (16 * db + 4 * (lane >> 4) + r) * NS + 16 * nb + (lane & 15)] = lam[jj][r];
      }
    }
  }
}

// dA[h, n] = sum over batch rows and runs of the per-run partials, in a fixed
// order: one workgroup per head, thread (g, n) sums partials g, g + G, ... in
// four interleaved accumulators (four loads in flight), then the G per-thread
// sums are added in order.  Per head (dA_sn == 0): dA[h] = the sum of those
// over n, in order of n.
template <int T>
__global__ __launch_bounds__(T) void ssd2_dA_kernel(const float* __restrict__ part, float* __restrict__ dA, int Bsz,
                                                    int H, int nR, int NS, int dA_sn) {
  __shared__ float red[T];
  const int h = blockIdx.x, G = T / NS, n = threadIdx.x % NS, g = threadIdx.x / NS;
  const int parts = Bsz * nR;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (g < G) {
    for (int i0 = g; i0 < parts; i0 += 4 * G) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = i0 + q * G;
        if (i < parts) {
          const int b = i / nR, r = i % nR;
          acc[q] += part[(((int64_t)b * H + h) * nR + r) * NS + n];
        }
      }
    }
  }
  red[threadIdx.x] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  __syncthreads();
  float t = 0.f;
  if (threadIdx.x < NS) {
    for (int q = 0; q < G; ++q) t += red[q * NS + threadIdx.x];
    if (dA_sn != 0) dA[(int64_t)h * NS + threadIdx.x] = t;
  }
  if (dA_sn == 0) {
    __syncthreads();   // every partial read; red[] takes the per-n sums
    if (threadIdx.x < NS) red[threadIdx.x] = t;
    __syncthreads();
    if (threadIdx.x == 0) {
      float s = 0.f;
      for (int n2 = 0; n2 < NS; ++n2) s += red[n2];
      dA[h] = s;
    }
  }
}

int launch_dA(const rr::ChunkArgs& p, int64_t B, hipStream_t s) {
  const int nR = (p.nC + p.R - 1) / p.R;   // runs per head
  // (a larger workgroup where the smaller one would leave a thread more than
  // four partials: more than one round of dependent loads, which come from
  // other XCDs' writes.  Dh 128 / N 64 at B3 L512: 3072 partials per head,
  // 3.96 µs with 256 threads)
  if ((int64_t)B * nR * p.NS > 1024)
    hipLaunchKernelGGL(ssd2_dA_kernel<1024>, dim3(p.H), dim3(1024), 0, s, p.ws, p.dA, (int)B, p.H, nR, p.NS, p.dA_sn);
  else
    hipLaunchKernelGGL(ssd2_dA_kernel<256>, dim3(p.H), dim3(256), 0, s, p.ws, p.dA, (int)B, p.H, nR, p.NS, p.dA_sn);
  return rr::check_launch("ssd chunked backward dA");
}

template <int DH, int NS>
int launch_bwd(const rr::ChunkArgs& p, int64_t B, hipStream_t s) {
  if (p.mode == kPipe) {   // R == 1
    if (int rc = rr::chunked::launch_scan<DH, NS, false>(p, B, s, true)) return rc;
    hipLaunchKernelGGL((ssd2_bwd_kernel<DH, NS, kPipe>), rr::chunked::chunk_grid(p), dim3(256), 0, s, p);
  } else if (p.mode == kSum || p.mode == kDirect) {   // R == 1; adjoint summed in the kernel
    hipLaunchKernelGGL((ssd2_bwd_kernel<DH, NS, kSum>), rr::chunked::chunk_grid(p), dim3(256), 0, s, p);
  } else {   // R == nC
    hipLaunchKernelGGL((ssd2_bwd_kernel<DH, NS, kWhole>), dim3(1, p.H, (unsigned)B), dim3(256), 0, s, p);
  }
  if (int rc = rr::check_launch("ssd chunked backward")) return rc;
  return launch_dA(p, B, s);
}

}  // namespace

namespace rr {

bool ssd2_bwd_supported(int64_t Dh, int64_t N) {
  if (Dh == 128) return N == 64 || N == 128;   // the column-owned kernel
  return (Dh == 32 || Dh == 64) && (N == 16 || N == 32 || N == 64 || N == 128);
}

// Wider states (N >= 64: the column-owned backward) take the direct mode only
// for the shortest heads.
constexpr int64_t kDirectMaxChunksWide = 4;
constexpr int64_t kDirectMaxWorkgroups = 4096;
// Dh 128 with N 64 (the reference's production shape) in short heads, few of
// them: the direct mode with block-owned sums (direct_sum_wide) while every
// chunk's workgroup can be resident at once (three per CU).
constexpr int64_t kWideDirectMaxWorkgroups = 3 * 256;
bool wide_direct(int64_t B, int64_t H, int64_t nC, int64_t Dh, int64_t N) {
  return Dh == 128 && N == 64 && nC <= chunked::kDirectMaxChunks && B * H * nC <= kWideDirectMaxWorkgroups;
}

int chunked_mode(int64_t B, int64_t H, int64_t nC, int64_t Dh, int64_t N, int pass) {
  const int64_t grid = nC * ((B * H + chunked::kXcds - 1) / chunked::kXcds * chunked::kXcds);
  if (grid >= ((int64_t)1 << 31)) return chunked::kWhole;   // beyond a 1-D per-chunk grid
  // Enough heads to fill the GPU: the forward runs whole heads; the backward
  // stays per chunk (measured on MI355X, fwd / bwd µs, whole-head vs per chunk:
  // B96 L512 H12 Dh64 N16 137 / 414 vs 194 / 357 (sum mode); B8 L4096 H80
  // Dh64 N128 2308 / 7457 vs 4025 / 4873 (pipelined)).
  if (B * H >= 512 && pass == 0) return chunked::kWhole;
  if (wide_direct(B, H, nC, Dh, N)) return chunked::kDirect;
  // Short heads: the forward holds all chunks of a head in one workgroup per
  // 16-column slice of d (no re-reads, no cross-workgroup carry)
  if (pass == 0 && res_fwd_supported(B, H, nC, Dh, N)) return chunked::kRes;
  // Short heads, few of them: every chunk's workgroup sums over the other
  // chunks' inputs itself (a single kernel per pass; the sums' reads grow as
  // nC^2 per head, so not once the workgroups fill the GPU several times
  // over); kSum where the backward's small-N kernel takes it (its forward is
  // the direct kernel)
  if (nC <= chunked::kDirectMaxChunks && N <= 32 && B * H * nC <= kDirectMaxWorkgroups) return chunked::kSum;
  if (nC <= kDirectMaxChunksWide && Dh * N <= chunked::kDirectMaxState) return chunked::kDirect;
  // Wide states (the column-owned backward) with the per-head adjoint scan:
  // a workgroup per pair of chunks, half the adjoints through memory
  // (measured at config 4: runs of 2 3.98 ms against 4.45 ms per chunk; runs
  // of 4 3.92 ms, but the carried adjoint's rounding then reaches 8e-6 of dA
  // where pairs keep 6e-6, so pairs)
  if (pass == 1 && N >= 64 && Dh <= 64 && nC % 2 == 0 && B * H >= chunked::kScanMinHeads)
    return chunked::kPair;
  return chunked::kPipe;
}

// Chunks per workgroup (ChunkArgs::R) of a mode.
int chunked_run(int mode, int64_t nC) {
  if (mode == chunked::kWhole) return (int)nC;
  if (mode == chunked::kPair) return 2;
  return 1;
}

// Workspace layout (floats, each part 256-byte aligned): per-chunk decays
// [B,H,nC] (pipelined mode), dA partials [B,H,nR,N] (backward), backward
// chunk aggregates / adjoints [B,H,nC,Dh,N] (pipelined backward; the wide
// direct mode's adjoints, which du's operands are read back from).
namespace {
int64_t align64(int64_t n) { return (n + 63) / 64 * 64; }
bool adjoint_slots(int mode, int64_t Dh, int64_t N) {
  return mode == chunked::kPipe || mode == chunked::kPair ||
         (mode == chunked::kDirect && Dh * N > chunked::kDirectMaxState);
}
}  // namespace

size_t ssd2_ws_bytes(int64_t B, int64_t H, int64_t nC, int mode, int64_t Dh, int64_t N, int pass) {
  const int64_t R = chunked_run(mode, nC), nR = (nC + R - 1) / R;
  const bool pipe = mode == chunked::kPipe || mode == chunked::kPair;
  int64_t f = pipe ? align64(B * H * nC) : 0;
  if (pass == 1) {
    f += align64(B * H * nR * N);
    if (adjoint_slots(mode, Dh, N)) f += align64(B * H * nR * Dh * N);   // one adjoint per run
  }
  return (size_t)f * sizeof(float);
}

void ssd2_carve_ws(ChunkArgs& a, void* ws, int64_t B, int pass) {
  float* f = static_cast<float*>(ws);
  const int64_t nR = (a.nC + a.R - 1) / a.R;
  const bool pipe = a.mode == chunked::kPipe || a.mode == chunked::kPair;
  a.tot = a.ws = a.agg = nullptr;
  if (pipe) { a.tot = f; f += align64(B * a.H * a.nC); }
  if (pass == 1) {
    a.ws = f; f += align64(B * a.H * nR * a.NS);
    if (adjoint_slots(a.mode, a.DH, a.NS)) a.agg = f;
  }
}

int64_t ssd2_ws_extent(int64_t B, int64_t H, int64_t nC, int mode, int64_t Dh, int64_t N, int pass) {
  using namespace chunked;
  ChunkArgs a{};
  a.B = (int)B; a.H = (int)H; a.nC = (int)nC; a.DH = (int)Dh; a.NS = (int)N; a.mode = mode;
  a.R = chunked_run(mode, nC);
  // carve from a stand-in base address (never dereferenced) and measure offsets
  char* const base = reinterpret_cast<char*>(uintptr_t(1) << 44);
  ssd2_carve_ws(a, base, B, pass);
  int64_t ext = 0;
  auto touch = [&](const float* region, int64_t first, int64_t count) {
    if (region == nullptr) return;
    ext = std::max<int64_t>(ext, reinterpret_cast<const char*>(region + first + count) - base);
  };
  const int64_t state = Dh * N, BH = B * H;
  const bool pipe = mode == kPipe || mode == kPair;
  if (pipe && BH < kScanMinHeads) {
    // aggregate kernel and state / adjoint pass: per-chunk decays and states
    for (int64_t id = 0; id < chunk_grid_size(a.B, a.H, a.nC); ++id) {
      const ChunkId c = decode_chunk((int)id, a.B, a.H, a.nC, a.NS, false, false);
      if (!c.valid) continue;
      const int64_t bh = (int64_t)c.b * H + c.h;
      touch(a.tot, bh * nC + c.c, 1);
      if (pass == 1) touch(a.agg, adj_slot(bh, a.nC, 1, c.c) * state, state);
    }
  } else if (pipe && pass == 1) {
    // adjoint scan: the adjoint leaving every R-th chunk of each head
    for (int64_t bh = 0; bh < BH; ++bh)
      for (int c = 0; c < a.nC; ++c)
        if (a.R == 1 || c % a.R == a.R - 1) touch(a.agg, adj_slot(bh, a.nC, a.R, c / a.R) * state, state);
  }
  if (pass != 1) return ext;
  // the chunk kernels: the adjoint each reads, the dA partial each writes
  const int nR = mode == kWhole ? 1 : mode == kPair ? a.nC / a.R : a.nC;
  if (mode == kWhole) {
    for (int64_t bh = 0; bh < BH; ++bh) touch(a.ws, dA_slot(bh, nR, 0) * N, N);
  } else if (mode == kPair) {
    for (int64_t id = 0; id < run_grid_size(a.B, a.H, a.nC, a.R); ++id) {
      const ChunkId r = decode_run((int)id, a.B, a.H, a.nC, a.R, a.NS);
      if (!r.valid) continue;
      const int64_t bh = (int64_t)r.b * H + r.h;
      touch(a.agg, adj_slot(bh, a.nC, a.R, r.c) * state, state);
      touch(a.ws, dA_slot(bh, nR, r.c) * N, N);
    }
  } else {
    for (int64_t id = 0; id < chunk_grid_size(a.B, a.H, a.nC); ++id) {
      const ChunkId c = decode_chunk((int)id, a.B, a.H, a.nC, a.NS, mode == kSum || mode == kDirect, false);
      if (!c.valid) continue;
      const int64_t bh = (int64_t)c.b * H + c.h;
      if (adjoint_slots(mode, Dh, N)) touch(a.agg, adj_slot(bh, a.nC, 1, c.c) * state, state);
      touch(a.ws, dA_slot(bh, nR, c.c) * N, N);
    }
  }
  return ext;
}

int ssd2_bwd(const ChunkArgs& p, int64_t B, hipStream_t s) {
  switch (p.DH * 1000 + p.NS) {
    case 32016: return launch_bwd<32, 16>(p, B, s);
    case 32032: return launch_bwd<32, 32>(p, B, s);
    case 64016: return launch_bwd<64, 16>(p, B, s);
    case 64032: return launch_bwd<64, 32>(p, B, s);
    case 32064: case 32128: case 64064: case 64128: case 128064: case 128128:
      if (int rc = chunked_bwd_cols(p, B, s, false)) return rc;
      return launch_dA(p, B, s);
    default: return fail(RR_EUNSUPPORTED, "ssd chunked backward: unsupported (Dh, N)");
  }
}

}  // namespace rr
