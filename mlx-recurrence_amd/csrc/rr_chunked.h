// rr_chunked.h — the chunked (MFMA) form shared by SSD with a head-uniform
// decay rate and GLA: step scalars, the chunk-aggregate and state-pass
// kernels, and the forward kernel.  Included by ssd_chunked.hip and
// gla_chunked.hip; each instantiates what it launches.
//
// Both scans are, per (batch, head), the recurrence over a state h[d, n]
//     h_t = dec_t h_{t-1} + w_t u_t B_t^T,     y_t = h_t C_t
// with a scalar decay per step:
//     SSD (reference ssd.py:85-111): dec_t = exp(a delta_t), w_t = delta_t,
//         u = u, B = B_in, C = C_in, d = channel, n = state;
//     GLA (reference gla.py:78-100): dec_t = g_t, w_t = 1,
//         u = v, B = k, C = q, d = j (value index), n = i (key index).
// Within a 32-step chunk, with M[t, s] = dec_{s+1} ... dec_t (s <= t),
// gam_t = dec_0 ... dec_t and m31_s = M[31, s]:
//     Y     = (M o C B^T o w_s) U  +  diag(gam) C h_in^T
//     h_end = gam_31 h_in + U^T diag(m31 o w) B
// Every product is a bf16 MFMA: inputs are exact in bf16, fp32 factors are
// split into hi + lo bf16 halves (x = hi + lo + O(2^-17 |x|)).
//
// SSD forms its decays as exp(a (cd_t - cd_s)) of the in-chunk cumulative
// delta cd; GLA forms them as running products of the gates, so gates of any
// sign (and zero) are handled exactly.
#pragma once

#include "rr_common.h"
#include "rr_internal.h"
#include "rr_mfma.h"

namespace rr {
namespace chunked {

constexpr int Q = 32;      // chunk length (steps)
constexpr int PQ = Q + 8;  // LDS pitch (elements) of [*][s] arrays: 80 bytes

template <int DH, int NS>
struct Cfg {
  static constexpr int PN = NS + 8;          // LDS pitch of [*][n] arrays
  static constexpr int NBD = DH / 16, NBN = NS / 16, NB = NBD * NBN;
  static constexpr int NBW = (NB + 3) / 4;   // 16x16 state blocks per wave (4 waves)
  static constexpr int NYB = DH / 32;        // 32x32 output blocks of Y
};

// Row of element r of a 32x32 MFMA accumulator held by `lane` (its column is
// lane % 32).
__device__ __forceinline__ int r32row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// Inclusive prefix sum / product over lanes 0..31 and, separately, 32..63
// (DPP row shifts, then row 0 (2) hands its total to row 1 (3)).
__device__ __forceinline__ float prefix32(float v, int /*lane*/) { return prefix32_sum(v); }
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_one(float v) {   // 1 where the source lane is outside the row
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, 1.f), __builtin_bit_cast(int, v),
                                                               CTRL, ROWS, 0xF, false));
}
__device__ __forceinline__ float prefix_prod32(float v, int /*lane*/) {
  v *= dpp_one<0x111, 0xF>(v);   // row_shr:1
  v *= dpp_one<0x112, 0xF>(v);   // row_shr:2
  v *= dpp_one<0x114, 0xF>(v);   // row_shr:4
  v *= dpp_one<0x118, 0xF>(v);   // row_shr:8
  v *= dpp_one<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
  return v;
}
// Inclusive suffix product over lanes (lane..31) within each half-wave.
__device__ __forceinline__ float suffix_prod32(float v, int lane) {
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) {
    const float x = __shfl_down(v, o, 32);
    if ((lane & 31) + o < 32) v *= x;
  }
  return v;
}

// Step scalars of one chunk; lane s < 32 holds step s, whose raw step input
// `x` (SSD delta_s, GLA g_s) it passes in.  Lanes >= 32 must pass the neutral
// input (SSD 0, GLA 1).
struct StepScalars {
  float gam;   // decay over steps 0..s
  float m31;   // decay over steps s+1..31
  float w;     // input weight (SSD delta_s, GLA 1)
  float cd;    // SSD: cumulative delta over steps 0..s (GLA: unused)
  float tot;   // chunk decay gam_31 (every lane)
};

template <bool GLA>
__device__ __forceinline__ StepScalars step_scalars(float x, float a, int lane) {
  StepScalars r;
  if constexpr (GLA) {
    r.gam = prefix_prod32(x, lane);
    const float suf = suffix_prod32(x, lane);
    const float nxt = __shfl_down(suf, 1, 32);
    r.m31 = (lane & 31) < 31 ? nxt : 1.f;
    r.w = 1.f;
    r.cd = 0.f;
    r.tot = __shfl(r.gam, 31);
  } else {
    r.cd = prefix32(x, lane);
    const float c31 = __shfl(r.cd, 31);
    r.gam = __expf(a * r.cd);
    r.m31 = __expf(a * (c31 - r.cd));
    r.w = x;
    r.tot = __expf(a * c31);
  }
  return r;
}

// exp(x) where `keep`, else 0.  The exponential is formed in every lane and
// then selected: written as a conditional expression it would compile to a
// lane-divergent branch per element, which serialises the LDS reads and
// exponentials it guards.  (A dropped lane may overflow to +inf; the select
// discards it.)
__device__ __forceinline__ float masked_exp(bool keep, float x) {
  const float e = __expf(x);
  return keep ? e : 0.f;
}

// The 16 decays M[t, s] held by `lane` in the 32x32 accumulator layout
// (s = lane % 32, t = r32row(r, lane)), zero above the diagonal (s > t).
// SSD reads the cumulative deltas cd[], GLA the gates g[] (both in LDS).
template <bool GLA>
__device__ __forceinline__ void decay_block32(const float* cd_or_g, float a, int lane, float (&m)[16]) {
  const int s = lane & 31;
  if constexpr (GLA) {
    const int half = lane >> 5;
    float run = 0.f;
#pragma unroll
    for (int t = 0; t < Q; ++t) {
      const float g = cd_or_g[t];   // read in every lane (no branch around it)
      run = t < s ? 0.f : (t == s ? 1.f : run * g);
      if (((t >> 2) & 1) == half) m[4 * (t >> 3) + (t & 3)] = run;
    }
  } else {
    const float cds = cd_or_g[s];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = r32row(r, lane);
      m[r] = masked_exp(s <= t, a * (cd_or_g[t] - cds));
    }
  }
}

// Offset of state element (d, n) in a caller's initial state, final-state
// cotangent or initial-state gradient: SSD keeps them [d][n] like the
// checkpoints, GLA as S[i][j] = [n][d] (reference gla.py:321-329).
template <bool GLA, int DH, int NS>
__device__ __forceinline__ int state_off(int d, int n) {
  if constexpr (GLA) return n * DH + d;
  else return d * NS + n;
}

// Modes of the chunked kernels (ChunkArgs::mode):
//   kWhole  a head per workgroup, state / adjoint carried in registers;
//   kPipe   one workgroup per chunk; aggregate kernel, state-pass kernel
//           (pass_kernel), chunk kernel;
//   kDirect one workgroup per chunk forming its entering state from the raw
//           inputs of the other chunks (nC <= kDirectMaxChunks);
//   kSum    one workgroup per chunk forming its entering state from the
//           chunk aggregates (agg_sum): aggregate kernel, chunk kernel.
enum Mode { kWhole = 0, kPipe = 1, kDirect = 2, kSum = 3 };
// kSum reads up to nC - 1 aggregates per workgroup (quadratic in nC), so it
// serves the middle range of chunk counts; longer heads run kPipe.
constexpr int kSumMaxChunks = 16;

// Per-chunk kernels run on a 1-D grid of chunk_grid(p) workgroups.  The GPU
// hands workgroups to its 8 XCDs round-robin by linear index; the decode
// gives every chunk of a head the same XCD (x = index % 8), so whatever the
// head's workgroups share (inputs, checkpoints, adjoints) is cached in one L2.
// Where the chunks cost the same (kPipe, kWhole's aggregates), a head's
// chunks go out together.  Where they differ (kDirect and kSum sum over the
// other chunks), the chunk position is the slowest-varying part of the index
// and the costliest chunks of every head go out first (`late_first`: from the
// last chunk, for forward sums; else from chunk 0); the cheap ones then take
// the third slots of the CUs, which run slowest.
constexpr int kXcds = 8;
struct ChunkId {
  int c, h, b;
  bool valid;   // false for the padding workgroups of the last head group
};
__device__ __forceinline__ ChunkId chunk_id(const ChunkArgs& p, bool by_cost, bool late_first) {
  const int id = blockIdx.x, x = id % kXcds, slot = id / kXcds;
  const int groups = (p.B * p.H + kXcds - 1) / kXcds;   // head groups of 8
  const int cs = by_cost ? slot / groups : slot % p.nC;
  const int bh = (by_cost ? slot % groups : slot / p.nC) * kXcds + x;
  return ChunkId{late_first ? p.nC - 1 - cs : cs, bh % p.H, bh / p.H, bh < p.B * p.H};
}
inline dim3 chunk_grid(const ChunkArgs& p) {
  return dim3((unsigned)(p.nC * ((p.B * p.H + kXcds - 1) / kXcds) * kXcds));
}

// Per-head decay rate (SSD); GLA has none.
template <bool GLA>
__device__ __forceinline__ float head_rate(const ChunkArgs& p, int h) {
  if constexpr (GLA) return 0.f;
  else return p.A[(int64_t)h * p.A_stride_h];
}

// ------------------------------------------------------------------ pipelined mode
// Several workgroups per head.  Three kernels per pass:
//  1. agg_kernel, one workgroup per chunk k, writes the chunk's aggregate and its
//     decay tot_k = gam_31:
//       forward:  S_k = U_k^T diag(m31 o w) B_k, the state the chunk adds from
//                 a zero start (into checkpoint slot k; kSum: the workspace);
//       backward: G_k = (gam o dY_k)^T C_k, the adjoint the chunk sends back to
//                 its start (into the workspace).
//  2. pass_kernel, one thread per state element, walks the chunks in order:
//       forward:  h_k = tot_k h_{k-1} + S_k   (h_{-1} = h0), into slot k
//       backward: lam_k = adjoint of the state leaving chunk k,
//                 lam_{nC-1} = dfinal, lam_{k-1} = tot_k lam_k + G_k,
//                 and dh0 = tot_0 lam_0 + G_0.
//  3. the main kernel, one workgroup per chunk, reads its entering state
//     (and, backward, lam_k) and does the chunk's dense products.
// agg_kernel: a workgroup of four waves per chunk stages the operands (all
// loads first), then wave w forms the 16x16 blocks j = w, w + 4, ... of the
// aggregate.
constexpr int kAggThreads = 256;
template <int DH, int NS, bool GLA>
__global__ __launch_bounds__(kAggThreads) void agg_kernel(ChunkArgs p, int kind) {
  constexpr int NBN = NS / 16, NB = (DH / 16) * NBN;
  __shared__ uint16_t XT_hi[DH][PQ], XT_lo[DH][PQ];   // kind 0: U^T [d][s] (hi only); kind 1: (gam o dY)^T
  __shared__ uint16_t YT_hi[NS][PQ], YT_lo[NS][PQ];   // kind 0: (m31 o w o B)^T split; kind 1: C^T (hi only)
  __shared__ float wsh[Q];                            // kind 0: m31_s w_s; kind 1: gam_t
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const ChunkId id = chunk_id(p, false, false);
  if (!id.valid) return;
  const int c = id.c, h = id.h, b = id.b;
  const float a = head_rate<GLA>(p, h);
  const int64_t rowH = p.H, row0 = (int64_t)b * p.L + (int64_t)c * Q;
  constexpr int T = kAggThreads;
  constexpr int UV = (Q * DH / 8 + T - 1) / T, GV = (Q * DH / 4 + T - 1) / T, BV = (Q * NS / 8 + T - 1) / T;
  // loads first
  u16x8_t uv[UV], bv[BV];
  float4 gv[GV];
  if (kind == 0) {
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + T * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
      uv[v] = i < Q * DH / 8 ? *reinterpret_cast<const u16x8_t*>(p.u + ((row0 + tl) * rowH + h) * DH + d0) : u16x8_t{};
    }
  } else {
#pragma unroll
    for (int v = 0; v < GV; ++v) {
      const int i = tid + T * v, tl = (i / (DH / 4)) & (Q - 1), d0 = 4 * (i % (DH / 4));
      gv[v] = i < Q * DH / 4 ? *reinterpret_cast<const float4*>(p.dy + ((row0 + tl) * rowH + h) * DH + d0)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  const uint16_t* bsrc = kind == 0 ? p.Bm : p.Cm;
#pragma unroll
  for (int v = 0; v < BV; ++v) {
    const int i = tid + T * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
    bv[v] = i < Q * NS / 8 ? *reinterpret_cast<const u16x8_t*>(bsrc + ((row0 + tl) * rowH + h) * NS + n0) : u16x8_t{};
  }
  if (w == 0) {
    const float xl = bf_val(p.delta[(row0 + (lane & (Q - 1))) * rowH + h]);   // unconditional load
    const float xv = lane < Q ? xl : (GLA ? 1.f : 0.f);
    const StepScalars sc = step_scalars<GLA>(xv, a, lane);
    if (lane < Q) wsh[lane] = kind == 0 ? sc.m31 * sc.w : sc.gam;
    if (lane == 0) p.tot[((int64_t)b * p.H + h) * p.nC + c] = sc.tot;
  }
  __syncthreads();
  if (kind == 0) {
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + T * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
      if (i < Q * DH / 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) XT_hi[d0 + e][tl] = uv[v][e];
      }
    }
  } else {
#pragma unroll
    for (int v = 0; v < GV; ++v) {
      const int i = tid + T * v, tl = (i / (DH / 4)) & (Q - 1), d0 = 4 * (i % (DH / 4));
      if (i < Q * DH / 4) {
        const float gt = wsh[tl];
        const float g4[4] = {gv[v].x, gv[v].y, gv[v].z, gv[v].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint16_t hi, lo;
          bf_split(gt * g4[e], hi, lo);
          XT_hi[d0 + e][tl] = hi;
          XT_lo[d0 + e][tl] = lo;
        }
      }
    }
  }
#pragma unroll
  for (int v = 0; v < BV; ++v) {
    const int i = tid + T * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
    if (i < Q * NS / 8) {
      const float ws = wsh[tl];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (kind == 0) {
          uint16_t hi, lo;
          bf_split(ws * bf_val(bv[v][e]), hi, lo);
          YT_hi[n0 + e][tl] = hi;
          YT_lo[n0 + e][tl] = lo;
        } else {
          YT_hi[n0 + e][tl] = bv[v][e];
        }
      }
    }
  }
  __syncthreads();
  float* dst = (kind == 0 && p.mode != kSum ? p.ckpt : p.agg) + (((int64_t)b * p.H + h) * p.nC + c) * DH * NS;
#pragma unroll
  for (int jj = 0; jj < (NB + 3) / 4; ++jj) {
    const int j = w + 4 * jj;
    if (j >= NB) break;
    const int db = j / NBN, nb = j % NBN;
    const u16x8_t fa = frag(&XT_hi[16 * db + (lane & 15)][8 * (lane >> 4)]);
    const u16x8_t fb = frag(&YT_hi[16 * nb + (lane & 15)][8 * (lane >> 4)]);
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = mfma16(fa, fb, acc);
    if (kind == 0) acc = mfma16(fa, frag(&YT_lo[16 * nb + (lane & 15)][8 * (lane >> 4)]), acc);
    else acc = mfma16(frag(&XT_lo[16 * db + (lane & 15)][8 * (lane >> 4)]), fb, acc);
#pragma unroll
    for (int r = 0; r < 4; ++r) dst[(16 * db + 4 * (lane >> 4) + r) * NS + 16 * nb + (lane & 15)] = acc[r];
  }
}

// Sequential pass over the chunks of one (batch, head), one state element per
// thread; loads are issued kPass chunks ahead of their use.
template <int DH, int NS, bool GLA>
__global__ __launch_bounds__(256) void pass_kernel(ChunkArgs p, int kind) {
  constexpr int kPass = 16;
  const int e = blockIdx.x * 256 + threadIdx.x;   // element d * NS + n
  const int es = state_off<GLA, DH, NS>(e / NS, e % NS);
  const int h = blockIdx.y, b = blockIdx.z;
  const int64_t bh = (int64_t)b * p.H + h;
  const float* tot = p.tot + bh * p.nC;
  const int nC = p.nC;
  if (kind == 0) {
    float* buf = p.ckpt + bh * nC * (DH * NS) + e;
    float x = p.h0 != nullptr ? p.h0[bh * DH * NS + es] : 0.f;
    for (int k0 = 0; k0 < nC; k0 += kPass) {
      float sv[kPass], tv[kPass];
#pragma unroll
      for (int q = 0; q < kPass; ++q) {
        const bool ok = k0 + q < nC;
        sv[q] = ok ? buf[(int64_t)(k0 + q) * DH * NS] : 0.f;
        tv[q] = ok ? tot[k0 + q] : 0.f;
      }
#pragma unroll
      for (int q = 0; q < kPass; ++q) {
        if (k0 + q < nC) {
          x = tv[q] * x + sv[q];
          buf[(int64_t)(k0 + q) * DH * NS] = x;
        }
      }
    }
  } else {
    float* buf = p.agg + bh * nC * (DH * NS) + e;
    float x = p.dfinal != nullptr ? p.dfinal[bh * DH * NS + es] : 0.f;
    for (int k0 = nC - 1; k0 >= 0; k0 -= kPass) {
      float gv[kPass], tv[kPass];
#pragma unroll
      for (int q = 0; q < kPass; ++q) {
        const bool ok = k0 - q >= 0;
        gv[q] = ok ? buf[(int64_t)(k0 - q) * DH * NS] : 0.f;
        tv[q] = ok ? tot[k0 - q] : 0.f;
      }
#pragma unroll
      for (int q = 0; q < kPass; ++q) {
        if (k0 - q >= 0) {
          buf[(int64_t)(k0 - q) * DH * NS] = x;
          x = tv[q] * x + gv[q];
        }
      }
    }
    if (p.dh0 != nullptr) p.dh0[bh * DH * NS + es] = x;
  }
}

// ------------------------------------------------------------------ sum mode
// Folds the aggregates k0 .. k0 + KB - 1 of the run (chunk j(k) = k, or
// nC - 1 - k backwards) into x.  All KB loads go out before the fold; the
// surplus ones past `cnt` repeat the last needed chunk's addresses (cache
// hits, dropped in the fold), so no branch waits on a load.
template <int DH, int NS, bool BWD, bool TRANS, int NX, int KB>
__device__ __forceinline__ void agg_fold(const ChunkArgs& p, const float* ag, const float* tt, int k0, int cnt,
                                         const int (&off)[NX], const bool (&has)[NX], f32x4_t (&x)[NX]) {
  float tv[KB];
  f32x4_t v[KB][NX];
#pragma unroll
  for (int k = 0; k < KB; ++k) {
    const int kk = min(k0 + k, cnt - 1);
    const int j = BWD ? p.nC - 1 - kk : kk;
    tv[k] = tt[j];
#pragma unroll
    for (int q = 0; q < NX; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[k][q][r] = ag[(int64_t)j * DH * NS + off[q] + (TRANS ? r : r * NS)];
  }
#pragma unroll
  for (int k = 0; k < KB; ++k) {
    const bool ok = k0 + k < cnt;
#pragma unroll
    for (int q = 0; q < NX; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) x[q][r] = ok && has[q] ? tv[k] * x[q][r] + v[k][q][r] : x[q][r];
  }
}

// kSum: the state entering chunk c (forward) or the adjoint leaving it
// (backward), from the chunk aggregates in p.agg and decays in p.tot by
// Horner's rule (the recursion pass_kernel runs, restricted to one chunk):
//   forward:  x = h0;     x = tot_j x + S_j  for j = 0 .. c - 1
//   backward: x = dfinal; x = tot_j x + G_j  for j = nC - 1 .. c + 1
// for this lane's elements of the 16x16 blocks (db(j), nb(j)) listed by
// `blk`, in the caller's register layout: element r at d = 16 db + 4 (lane / 16)
// + r, n = 16 nb + lane % 16 (TRANS false), or at d = 16 db + lane % 16,
// n = 16 nb + 4 (lane / 16) + r (TRANS true).  The number of aggregates is
// uniform over the workgroup; a batch of 4, 8 or 16 (as registers allow)
// covers it, so a workgroup reads little beyond the aggregates it needs.
template <int DH, int NS, bool GLA, bool BWD, bool TRANS = false, int NX, typename BLK>
__device__ __forceinline__ void agg_sum(const ChunkArgs& p, int c, int64_t bh, int lane, BLK blk,
                                        f32x4_t (&x)[NX]) {
  constexpr int kBatch = NX == 1 ? 16 : NX == 2 ? 8 : 4;
  const float* ext = BWD ? p.dfinal : p.h0;
  int off[NX];
  bool has[NX];
#pragma unroll
  for (int q = 0; q < NX; ++q) {
    int db, nb;
    has[q] = blk(q, db, nb);
    off[q] = !has[q] ? 0
             : TRANS ? (16 * db + (lane & 15)) * NS + 16 * nb + 4 * (lane >> 4)
                     : (16 * db + 4 * (lane >> 4)) * NS + 16 * nb + (lane & 15);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = off[q] + (TRANS ? r : r * NS), d = e / NS, n = e % NS;
      x[q][r] = has[q] && ext != nullptr ? ext[bh * DH * NS + state_off<GLA, DH, NS>(d, n)] : 0.f;
    }
  }
  const float* ag = p.agg + bh * p.nC * DH * NS;
  const float* tt = p.tot + bh * p.nC;
  const int cnt = BWD ? p.nC - 1 - c : c;
  if (cnt <= 0) return;
  if (cnt <= 4) {
    agg_fold<DH, NS, BWD, TRANS, NX, 4>(p, ag, tt, 0, cnt, off, has, x);
  } else if (kBatch >= 8 && cnt <= 8) {
    agg_fold<DH, NS, BWD, TRANS, NX, (kBatch >= 8 ? 8 : 4)>(p, ag, tt, 0, cnt, off, has, x);
  } else {
    for (int k0 = 0; k0 < cnt; k0 += kBatch) agg_fold<DH, NS, BWD, TRANS, NX, kBatch>(p, ag, tt, k0, cnt, off, has, x);
  }
}

// ------------------------------------------------------------------ direct mode
// Short sequences (nC <= kDirectMaxChunks): one workgroup per chunk forms the
// state entering its chunk (forward) or the adjoint leaving it (backward)
// itself, as a weighted sum over the inputs of all earlier (later) chunks, so
// a pass is a single kernel with no aggregate or state-pass kernels:
//   forward:  h_in(c) = Gam h0 + sum_{j<c} F_j U_j^T diag(m31 o w) B_j,
//             F_j = tot_{j+1} ... tot_{c-1},   Gam = tot_0 ... tot_{c-1};
//   backward: lam(c) = Gam dfinal + sum_{j>c} F_j (gam o dY_j)^T C_j,
//             F_j = tot_{c+1} ... tot_{j-1},   Gam = tot_{c+1} ... tot_{nC-1}
// (m31, w, gam and tot of chunk j as in step_scalars).  Wave w takes chunks
// w, w + 4, ... of the range and accumulates every 16x16 block of the state;
// the four partial sums are added in a fixed order (deterministic).
// The sum costs each workgroup up to nC - 1 chunks of extra reads; measured on
// MI355X (B3 H12 Dh64), it beats the two extra launches of the pipelined mode
// at 2 and 4 chunks and loses from 8 chunks on.
constexpr int kDirectMaxChunks = 4;
constexpr int kDirectMaxState = 64 * 64;   // Dh * N (the partial sums live in LDS)
constexpr int kDirectPerWave = kDirectMaxChunks / 4;

template <int DH, int NS, bool BWD>
struct DirectSmem {
  union {
    struct {                                // one wave's staging area
      uint16_t XT[BWD ? 2 : 1][DH][PQ];     // fwd: U^T; bwd: (coef o dY)^T hi, lo
      uint16_t YT[BWD ? 1 : 2][NS][PQ];     // fwd: (coef o B)^T hi, lo; bwd: C^T
    } st[4];
    float red[4][DH * NS];                  // per-wave partial sums, [d][n]
  };
  float tot[kDirectMaxChunks];
};

// Runs the weighted sum; afterwards red[] holds the four partial sums and the
// return value is Gam.  Every thread of the (256-thread) workgroup must call it.
template <int DH, int NS, bool GLA, bool BWD>
__device__ float direct_sum(const ChunkArgs& p, int c, int b, int h, float a, DirectSmem<DH, NS, BWD>& s) {
  constexpr int NBN = NS / 16, NB = (DH / 16) * NBN;
  constexpr int XV = BWD ? Q * DH / 4 / 64 : Q * DH / 8 / 64;  // float4 (dY) or u16x8 (U) per lane
  constexpr int YV = (Q * NS / 8 + 63) / 64;                   // u16x8 of B (fwd) or C (bwd) per lane
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l15 = lane & 15, l4 = lane >> 4;
  const int64_t rowH = p.H;
  const int j0 = BWD ? c + 1 : 0, j1 = BWD ? p.nC : c;   // chunks [j0, j1)
  const float neutral = GLA ? 1.f : 0.f;

  // 1. decays of the chunks in the range; per-step coefficients of this wave's
  float coef[kDirectPerWave];
#pragma unroll
  for (int jj = 0; jj < kDirectPerWave; ++jj) {
    const int j = j0 + w + 4 * jj;
    coef[jj] = 0.f;
    if (j < j1) {
      const int64_t row0 = (int64_t)b * p.L + (int64_t)j * Q;
      const float xl = bf_val(p.delta[(row0 + (lane & (Q - 1))) * rowH + h]);   // unconditional load
      const float xv = lane < Q ? xl : neutral;
      const StepScalars sc = step_scalars<GLA>(xv, a, lane);
      coef[jj] = BWD ? sc.gam : sc.m31 * sc.w;
      if (lane == 0) s.tot[j - j0] = sc.tot;
    }
  }
  __syncthreads();
  float gam_all = 1.f;
  for (int k = j0; k < j1; ++k) gam_all *= s.tot[k - j0];
#pragma unroll
  for (int jj = 0; jj < kDirectPerWave; ++jj) {
    const int j = j0 + w + 4 * jj;
    if (j < j1) {
      float f = 1.f;
      const int kb = BWD ? j0 : j + 1, ke = BWD ? j : j1;
      for (int k = kb; k < ke; ++k) f *= s.tot[k - j0];
      coef[jj] *= f;
    }
  }

  // 2. this wave's partial sum over its chunks (inputs of chunk jj + 1 are
  //    loaded while chunk jj is staged and multiplied)
  f32x4_t part[NB];
#pragma unroll
  for (int q = 0; q < NB; ++q) part[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto& st = s.st[w];
  const uint16_t* ysrc = BWD ? p.Cm : p.Bm;
  u16x8_t xu[2][BWD ? 1 : XV], yv[2][YV];
  float4 xf[2][BWD ? XV : 1];
  auto load = [&](int buf, int j) {
    const int64_t row0 = (int64_t)b * p.L + (int64_t)j * Q;
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      if constexpr (BWD) {
        const int i = lane + 64 * v, tl = i / (DH / 4), d0 = 4 * (i % (DH / 4));
        xf[buf][v] = *reinterpret_cast<const float4*>(p.dy + ((row0 + tl) * rowH + h) * DH + d0);
      } else {
        const int i = lane + 64 * v, tl = i / (DH / 8), d0 = 8 * (i % (DH / 8));
        xu[buf][v] = *reinterpret_cast<const u16x8_t*>(p.u + ((row0 + tl) * rowH + h) * DH + d0);
      }
    }
#pragma unroll
    for (int v = 0; v < YV; ++v) {
      const int i = lane + 64 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
      yv[buf][v] = i < Q * NS / 8 ? *reinterpret_cast<const u16x8_t*>(ysrc + ((row0 + tl) * rowH + h) * NS + n0)
                                  : u16x8_t{};
    }
  };
  if (j0 + w < j1) load(0, j0 + w);
#pragma unroll
  for (int jj = 0; jj < kDirectPerWave; ++jj) {
    const int j = j0 + w + 4 * jj;
    if (j >= j1) break;
    const int cur = jj & 1;
    if (j + 4 < j1) load(cur ^ 1, j + 4);
    const float cf = coef[jj];
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      if constexpr (BWD) {
        const int i = lane + 64 * v, tl = i / (DH / 4), d0 = 4 * (i % (DH / 4));
        const float ct = __shfl(cf, tl);
        const float g4[4] = {xf[cur][v].x, xf[cur][v].y, xf[cur][v].z, xf[cur][v].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint16_t hi, lo;
          bf_split(ct * g4[e], hi, lo);
          st.XT[0][d0 + e][tl] = hi;
          st.XT[BWD ? 1 : 0][d0 + e][tl] = lo;
        }
      } else {
        const int i = lane + 64 * v, tl = i / (DH / 8), d0 = 8 * (i % (DH / 8));
#pragma unroll
        for (int e = 0; e < 8; ++e) st.XT[0][d0 + e][tl] = xu[cur][v][e];
      }
    }
#pragma unroll
    for (int v = 0; v < YV; ++v) {
      const int i = lane + 64 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
      const float ct = __shfl(cf, tl);
      if (i < Q * NS / 8) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (BWD) {
            st.YT[0][n0 + e][tl] = yv[cur][v][e];
          } else {
            uint16_t hi, lo;
            bf_split(ct * bf_val(yv[cur][v][e]), hi, lo);
            st.YT[0][n0 + e][tl] = hi;
            st.YT[BWD ? 0 : 1][n0 + e][tl] = lo;
          }
        }
      }
    }
    wave_lds_sync();
#pragma unroll
    for (int q = 0; q < NB; ++q) {
      const int db = q / NBN, nb = q % NBN;
      const u16x8_t fa = frag(&st.XT[0][16 * db + l15][8 * l4]);
      const u16x8_t fb = frag(&st.YT[0][16 * nb + l15][8 * l4]);
      part[q] = mfma16(fa, fb, part[q]);
      if constexpr (BWD) part[q] = mfma16(frag(&st.XT[BWD ? 1 : 0][16 * db + l15][8 * l4]), fb, part[q]);
      else part[q] = mfma16(fa, frag(&st.YT[BWD ? 0 : 1][16 * nb + l15][8 * l4]), part[q]);
    }
    wave_lds_sync();
  }
  // 3. partial sums to LDS (the staging areas are dead once every wave is here)
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NB; ++q) {
    const int db = q / NBN, nb = q % NBN;
#pragma unroll
    for (int r = 0; r < 4; ++r) s.red[w][(16 * db + 4 * l4 + r) * NS + 16 * nb + l15] = part[q][r];
  }
  __syncthreads();
  return gam_all;
}

// Element (d, n) of the direct sum: the four partials plus Gam times the
// caller's h0 (forward) or dfinal (backward), read from red[] / `ext`.
template <int DH, int NS, bool GLA, bool BWD>
__device__ __forceinline__ float direct_value(const DirectSmem<DH, NS, BWD>& s, float gam_all, const float* ext,
                                              int d, int n) {
  const int e = d * NS + n;
  float v = ((s.red[0][e] + s.red[1][e]) + s.red[2][e]) + s.red[3][e];
  if (ext != nullptr) v += gam_all * ext[state_off<GLA, DH, NS>(d, n)];
  return v;
}

// ------------------------------------------------------------------ forward
template <int DH, int NS>
struct FwdSmem {
  uint16_t Ut[DH][PQ];                 // U^T  [d][s]
  uint16_t C[Q][Cfg<DH, NS>::PN];      // C    [t][n]
  uint16_t B[Q][Cfg<DH, NS>::PN];      // B    [s][n]
  uint16_t BwT_hi[NS][PQ];             // (m31 o w o B)^T [n][s]
  uint16_t BwT_lo[NS][PQ];
  uint16_t W_hi[Q][PQ];                // M o CB^T o w_s  [t][s]
  uint16_t W_lo[Q][PQ];
  float x[Q];      // step input (SSD delta, GLA gate)
  float cd[Q];     // SSD: cumulative delta
  float gam[Q];
};

template <int DH, int NS, bool DIRECT>
union FwdShared {
  FwdSmem<DH, NS> f;
};
template <int DH, int NS>
union FwdShared<DH, NS, true> {
  FwdSmem<DH, NS> f;
  DirectSmem<DH, NS, false> d;
};

// One chunk per workgroup with the entering state from checkpoint slot c - 1
// (kPipe, written by pass_kernel), from the direct sum (kDirect) or from the
// aggregates (kSum); or a run of R = nC chunks per workgroup carrying the
// state in registers (kWhole).
//
// Wave w owns the state rows d of the 16-row blocks db = w, w + 4, ... and
// holds them transposed in registers: block (db, nb), element r at
// n = 16 nb + 4 (lane / 16) + r, d = 16 db + lane % 16 — which is, element for
// element, the B operand of v_mfma_f32_16x16x16_bf16 contracting over n (the
// C h_in^T term of Y) and the accumulator of the state update
// h^T += (m31 o w o B)^T U.  So every wave forms Y and the new state of its
// rows with no cross-wave sum and no LDS copy of the state:
//   Y[t, d] = (W U)[t, d] + gam_t (C h_in^T)[t, d],  W = M o C B^T o w_s
//   h_end^T = gam_31 h_in^T + (m31 o w o B)^T U
template <int DH, int NS, int MODE, bool GLA>
__global__ __launch_bounds__(256) void fwd_kernel(ChunkArgs p) {
  using K = Cfg<DH, NS>;
  constexpr int NBD = DH / 16, NBN = NS / 16;
  constexpr int DBW = (NBD + 3) / 4;   // row blocks per wave
  constexpr bool STATE = MODE == kWhole || MODE == kDirect;   // forms the chunk's end state
  __shared__ FwdShared<DH, NS, MODE == kDirect> smu;
  auto& sm = smu.f;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l15 = lane & 15, l4 = lane >> 4;
  int h, b, cbeg;
  if constexpr (MODE == kWhole) {
    h = blockIdx.y, b = blockIdx.z, cbeg = 0;
  } else {
    constexpr bool kSums = MODE == kDirect || MODE == kSum;   // late chunks cost most
    const ChunkId id = chunk_id(p, kSums, kSums);
    if (!id.valid) return;
    h = id.h, b = id.b, cbeg = id.c;
  }
  // one chunk per workgroup except in the whole-head mode (a visible single
  // iteration keeps the compiler from hoisting addresses out of the loop)
  const int cend = MODE == kWhole ? min(cbeg + p.R, p.nC) : cbeg + 1;
  const float a = head_rate<GLA>(p, h);
  const int64_t rowH = p.H, bh = (int64_t)b * p.H + h;

  f32x4_t hst[DBW][NBN];   // this wave's rows of the state, transposed blocks
#pragma unroll
  for (int i = 0; i < DBW; ++i)
#pragma unroll
    for (int nb = 0; nb < NBN; ++nb) hst[i][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if constexpr (MODE == kDirect) {
    const float gam_all = direct_sum<DH, NS, GLA, false>(p, cbeg, b, h, a, smu.d);
    const float* h0b = p.h0 != nullptr ? p.h0 + bh * DH * NS : nullptr;
#pragma unroll
    for (int i = 0; i < DBW; ++i) {
      const int db = w + 4 * i;
      if (db < NBD) {
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            hst[i][nb][r] = direct_value<DH, NS, GLA, false>(smu.d, gam_all, h0b, 16 * db + l15, 16 * nb + 4 * l4 + r);
      }
    }
    __syncthreads();   // the chunk below reuses the LDS of the sum
  } else if constexpr (MODE == kPipe || MODE == kWhole) {
    // entering state: checkpoint slot c - 1 ([d][n], four consecutive n per
    // lane: one 16-byte load) or h0
    const bool from_h0 = cbeg == 0;
    const float* hsrc = !from_h0 ? p.ckpt + (bh * p.nC + cbeg - 1) * DH * NS
                                 : (p.h0 != nullptr ? p.h0 + bh * DH * NS : nullptr);
    if (hsrc != nullptr) {
#pragma unroll
      for (int i = 0; i < DBW; ++i) {
        const int db = w + 4 * i;
        if (db < NBD) {
#pragma unroll
          for (int nb = 0; nb < NBN; ++nb) {
            const int d = 16 * db + l15, n0 = 16 * nb + 4 * l4;
            if (from_h0) {
#pragma unroll
              for (int r = 0; r < 4; ++r) hst[i][nb][r] = hsrc[state_off<GLA, DH, NS>(d, n0 + r)];
            } else {
              const float4 v = *reinterpret_cast<const float4*>(hsrc + d * NS + n0);
              hst[i][nb] = f32x4_t{v.x, v.y, v.z, v.w};
            }
          }
        }
      }
    }
  }

  for (int c = cbeg; c < cend; ++c) {
    // a fresh copy of the thread index per chunk keeps the compiler from
    // hoisting every per-lane address of the body out of the chunk loop
    int tidv = tid;
    if constexpr (MODE == kWhole) asm volatile("" : "+v"(tidv));
    const int tid = tidv, lane = tidv & 63, l15 = lane & 15, l4 = lane >> 4;
    const int64_t row0 = (int64_t)b * p.L + (int64_t)c * Q;  // first (b, t) row of the chunk
    // ---- stage the chunk's inputs (all loads issued before any use)
    {
      constexpr int UV = (Q * DH / 8 + 255) / 256, BV = (Q * NS / 8 + 255) / 256;
      u16x8_t uv[UV], bv[BV], cv[BV];
#pragma unroll
      for (int v = 0; v < UV; ++v) {
        const int i = tid + 256 * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
        uv[v] = i < Q * DH / 8 ? *reinterpret_cast<const u16x8_t*>(p.u + ((row0 + tl) * rowH + h) * DH + d0) : u16x8_t{};
      }
#pragma unroll
      for (int v = 0; v < BV; ++v) {
        const int i = tid + 256 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
        const int64_t g = ((row0 + tl) * rowH + h) * NS + n0;
        bv[v] = i < Q * NS / 8 ? *reinterpret_cast<const u16x8_t*>(p.Bm + g) : u16x8_t{};
        cv[v] = i < Q * NS / 8 ? *reinterpret_cast<const u16x8_t*>(p.Cm + g) : u16x8_t{};
      }
      // unconditional (in-bounds) load, so no branch waits on it
      const float xv = bf_val(p.delta[(row0 + (tid & (Q - 1))) * rowH + h]);
      if constexpr (MODE == kSum) {
        // entering state from the aggregates (their loads go out behind the
        // chunk's own); this workgroup writes checkpoint slot c - 1 (its
        // entering state) and the last one also slot nC - 1
        agg_sum<DH, NS, GLA, false, true>(p, cbeg, bh, lane, [&](int q, int& db, int& nb) {
          db = w + 4 * (q / NBN), nb = q % NBN;
          return db < NBD;
        }, reinterpret_cast<f32x4_t(&)[DBW * NBN]>(hst));
        const float* ag_last = p.agg + (bh * p.nC + p.nC - 1) * DH * NS;
        const float t_last = p.tot[bh * p.nC + p.nC - 1];
#pragma unroll
        for (int i = 0; i < DBW; ++i) {
          const int db = w + 4 * i;
          if (db < NBD) {
#pragma unroll
            for (int nb = 0; nb < NBN; ++nb) {
              const int e = (16 * db + l15) * NS + 16 * nb + 4 * l4;
              const f32x4_t v = hst[i][nb];
              if (cbeg > 0)
                *reinterpret_cast<float4*>(p.ckpt + (bh * p.nC + cbeg - 1) * DH * NS + e) =
                    make_float4(v[0], v[1], v[2], v[3]);
              if (cbeg == p.nC - 1) {
                const float4 g = *reinterpret_cast<const float4*>(ag_last + e);
                *reinterpret_cast<float4*>(p.ckpt + (bh * p.nC + cbeg) * DH * NS + e) =
                    make_float4(t_last * v[0] + g.x, t_last * v[1] + g.y, t_last * v[2] + g.z, t_last * v[3] + g.w);
              }
            }
          }
        }
      }
#pragma unroll
      for (int v = 0; v < UV; ++v) {
        const int i = tid + 256 * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
        if (i < Q * DH / 8) {
#pragma unroll
          for (int e = 0; e < 8; ++e) sm.Ut[d0 + e][tl] = uv[v][e];
        }
      }
#pragma unroll
      for (int v = 0; v < BV; ++v) {
        const int i = tid + 256 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
        if (i < Q * NS / 8) {
          *reinterpret_cast<u16x8_t*>(&sm.B[tl][n0]) = bv[v];
          *reinterpret_cast<u16x8_t*>(&sm.C[tl][n0]) = cv[v];
        }
      }
      if (tid < Q) sm.x[tid] = xv;
    }
    __syncthreads();
    // ---- step scalars (every wave; lanes s and s + 32 hold step s);
    // W = M o C B^T o w_s (wave 0); (m31 o w o B)^T (the other waves)
    const StepScalars sc = step_scalars<GLA>(sm.x[lane & (Q - 1)], a, lane);
    if (w == 0) {
      if (lane < Q) {
        sm.cd[lane] = sc.cd;
        sm.gam[lane] = sc.gam;
      }
      wave_lds_sync();   // cd for the decays below
      f32x16_t cb = {};
#pragma unroll
      for (int kb = 0; kb < NS / 16; ++kb)
        cb = mfma32(frag(&sm.C[lane & 31][16 * kb + 8 * (lane >> 5)]),
                    frag(&sm.B[lane & 31][16 * kb + 8 * (lane >> 5)]), cb);
      const int s = lane & 31;
      float m[16];
      decay_block32<GLA>(GLA ? sm.x : sm.cd, a, lane, m);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = r32row(r, lane);
        uint16_t hi, lo;
        bf_split(m[r] * sc.w * cb[r], hi, lo);
        sm.W_hi[t][s] = hi;
        sm.W_lo[t][s] = lo;
      }
    } else if constexpr (STATE) {
      // lane s (and s + 32) weights column s; 192 threads cover Q x NS
      const float wend = sc.m31 * sc.w;
      for (int i = tid - 64; i < Q * NS; i += 192) {
        const int n = i / Q, s = i % Q;
        uint16_t hi, lo;
        bf_split(wend * bf_val(sm.B[s][n]), hi, lo);
        sm.BwT_hi[n][s] = hi;
        sm.BwT_lo[n][s] = lo;
      }
    }
    __syncthreads();
    // ---- Y and the end state of this wave's rows
    const float Gam = sc.tot;
#pragma unroll
    for (int i = 0; i < DBW; ++i) {
      const int db = w + 4 * i;
      if (db >= NBD) continue;
      u16x4_t hh[NBN], hl[NBN];
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) rr::bf_split4(hst[i][nb], hh[nb], hl[nb]);
      const u16x8_t fu = frag(&sm.Ut[16 * db + l15][8 * l4]);   // U [s][d]: B operand, k = s
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        f32x4_t yi = {0.f, 0.f, 0.f, 0.f}, ye = {0.f, 0.f, 0.f, 0.f};
        yi = mfma16(frag(&sm.W_hi[16 * tb + l15][8 * l4]), fu, yi);
        yi = mfma16(frag(&sm.W_lo[16 * tb + l15][8 * l4]), fu, yi);
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          const u16x4_t fc = frag4(&sm.C[16 * tb + l15][16 * nb + 4 * l4]);
          ye = mfma16k16(fc, hh[nb], ye);
          ye = mfma16k16(fc, hl[nb], ye);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tb + 4 * l4 + r;
          p.y[((row0 + t) * rowH + h) * DH + 16 * db + l15] = yi[r] + sm.gam[t] * ye[r];
        }
      }
      if constexpr (STATE) {
        float* ck = p.ckpt + (bh * p.nC + c) * DH * NS;
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
          acc = mfma16(frag(&sm.BwT_hi[16 * nb + l15][8 * l4]), fu, acc);
          acc = mfma16(frag(&sm.BwT_lo[16 * nb + l15][8 * l4]), fu, acc);
#pragma unroll
          for (int r = 0; r < 4; ++r) hst[i][nb][r] = Gam * hst[i][nb][r] + acc[r];
          *reinterpret_cast<float4*>(ck + (16 * db + l15) * NS + 16 * nb + 4 * l4) =
              make_float4(hst[i][nb][0], hst[i][nb][1], hst[i][nb][2], hst[i][nb][3]);
        }
      }
    }
    if constexpr (MODE == kWhole) __syncthreads();   // the next chunk rewrites the LDS
  }
}

template <int DH, int NS, bool GLA>
int launch_fwd(const ChunkArgs& p, int64_t B, hipStream_t s) {
  if (p.mode == kPipe) {   // R == 1
    hipLaunchKernelGGL((agg_kernel<DH, NS, GLA>), chunk_grid(p), dim3(kAggThreads), 0, s, p, 0);
    if (int rc = check_launch("chunked forward aggregates")) return rc;
    hipLaunchKernelGGL((pass_kernel<DH, NS, GLA>), dim3(DH * NS / 256, p.H, (unsigned)B), dim3(256), 0, s, p, 0);
    if (int rc = check_launch("chunked forward state pass")) return rc;
    hipLaunchKernelGGL((fwd_kernel<DH, NS, kPipe, GLA>), chunk_grid(p), dim3(256), 0, s, p);
  } else if (p.mode == kSum) {   // R == 1
    hipLaunchKernelGGL((agg_kernel<DH, NS, GLA>), chunk_grid(p), dim3(kAggThreads), 0, s, p, 0);
    if (int rc = check_launch("chunked forward aggregates")) return rc;
    hipLaunchKernelGGL((fwd_kernel<DH, NS, kSum, GLA>), chunk_grid(p), dim3(256), 0, s, p);
  } else if (p.mode == kDirect) {   // R == 1
    if constexpr (DH * NS <= kDirectMaxState)
      hipLaunchKernelGGL((fwd_kernel<DH, NS, kDirect, GLA>), chunk_grid(p), dim3(256), 0, s, p);
    else
      return fail(RR_EUNSUPPORTED, "chunked forward: state too large for the direct mode");
  } else {   // R == nC
    hipLaunchKernelGGL((fwd_kernel<DH, NS, kWhole, GLA>), dim3(1, p.H, (unsigned)B), dim3(256), 0, s, p);
  }
  return check_launch("chunked forward");
}

}  // namespace chunked
}  // namespace rr
