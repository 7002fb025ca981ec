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

#include <type_traits>

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
// The value of lane `src` (a constant), in every lane (v_readlane).
__device__ __forceinline__ float lane_value(float v, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}
// Inclusive suffix product over lanes (lane..31) within each half-wave:
// row_shl shifts within each 16-lane row, then rows 0 and 2 take the totals
// of rows 1 and 3 (their first lanes).  No LDS-unit permutes.
__device__ __forceinline__ float suffix_prod32(float v, int lane) {
  v *= dpp_one<0x101, 0xF>(v);   // row_shl:1
  v *= dpp_one<0x102, 0xF>(v);   // row_shl:2
  v *= dpp_one<0x104, 0xF>(v);   // row_shl:4
  v *= dpp_one<0x108, 0xF>(v);   // row_shl:8
  const float r1 = lane_value(v, 16), r3 = lane_value(v, 48);
  const int row = lane >> 4;
  return row == 0 ? v * r1 : row == 2 ? v * r3 : v;
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
    // m31_s = g_{s+1} ... g_31: the suffix product of the inputs shifted by
    // one lane (lane 15 of each half takes lane 16's input across the row)
    float x1 = dpp_one<0x101, 0xF>(x);   // row_shl:1
    const float x16 = lane_value(x, 16), x48 = lane_value(x, 48);
    x1 = (lane & 31) == 15 ? (lane < 32 ? x16 : x48) : x1;
    r.m31 = suffix_prod32(x1, lane);
    r.w = 1.f;
    r.cd = 0.f;
    r.tot = lane_value(r.gam, 31);
  } else {
    r.cd = prefix32(x, lane);
    const float c31 = lane_value(r.cd, 31);
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
    // All 32 gates are read (and pinned) before the chain: a read that the
    // chain's selects need in only some lanes was otherwise moved into a
    // divergent branch per step, serialising 32 LDS round trips.
    float gv[Q];
#pragma unroll
    for (int t = 0; t < Q; ++t) gv[t] = cd_or_g[t];
#pragma unroll
    for (int t = 0; t < Q; ++t) pin(gv[t]);
    float run = 0.f;
#pragma unroll
    for (int t = 0; t < Q; ++t) {
      const float prod = run * gv[t];
      const float diag = t == s ? 1.f : prod;
      run = t < s ? 0.f : diag;
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
//   kDirect one workgroup per chunk forming its entering state (forward) or
//           leaving adjoint (backward) from the raw inputs of the other chunks
//           (direct_sum, or direct_sum_wide for states past kDirectMaxState;
//           nC <= kDirectMaxChunks): one kernel per pass;
//   kSum    the same sum, for the backward's small-N kernel (its own
//           instantiation); the forward runs the direct kernel.
// Both read up to nC - 1 chunks of inputs per workgroup (quadratic in nC), so
// they serve short heads; longer heads run kPipe.
//   kRes    forward only: every chunk of a head resident in one workgroup
//           per 16-column slice of d (resident.hip), nC <= 16;
//   kPair   backward of the column-owned kernel with the per-head adjoint
//           scan: one workgroup per run of R = 2 or 4 consecutive chunks;
//           the scan stores the adjoint leaving every R-th chunk only, and
//           the workgroup carries it across the run's inner boundaries.
enum Mode { kWhole = 0, kPipe = 1, kDirect = 2, kSum = 3, kRes = 4, kPair = 5 };

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
// Heads whose B / C rows share a 128-byte line: a step's row of one head is
// NS bf16 values, so G = 128 / (2 NS) consecutive heads read the same lines
// (N = 16: four heads per line).  Every read request fills a whole line, so
// such heads placed on different XCDs fetch each line once per XCD.
__host__ __device__ inline int line_heads(int NS) { return NS >= 64 ? 1 : 64 / NS; }
// The (batch * H + head) index of head group j (of `groups`, 8 heads each) on
// XCD x: runs of G consecutive heads on one XCD, as long as whole runs of G
// groups remain; the rest one head per XCD in turn.  A bijection of
// [0, 8 groups); every XCD gets `groups` heads, as with bh = 8 j + x.
__host__ __device__ inline int head_on_xcd(int j, int x, int groups, int G) {
  const int q = groups / G * G;
  return j < q ? G * (kXcds * (j / G) + x) + j % G : kXcds * j + x;
}
// Chunk (or, for kPair, run) of workgroup `id` of a per-chunk grid: the
// decode of chunk_id / run_id below, callable on the host so that the
// workspace bound (rr_ssd_workspace_extent) walks the grid the kernels run.
__host__ __device__ inline ChunkId decode_chunk(int id, int B, int H, int nC, int NS, bool by_cost, bool late_first) {
  const int x = id % kXcds, slot = id / kXcds;
  const int groups = (B * H + kXcds - 1) / kXcds;   // head groups of 8
  const int cs = by_cost ? slot / groups : slot % nC;
  const int bh = head_on_xcd(by_cost ? slot % groups : slot / nC, x, groups, line_heads(NS));
  return ChunkId{late_first ? nC - 1 - cs : cs, bh % H, bh / H, bh < B * H};
}
__host__ __device__ inline ChunkId decode_run(int id, int B, int H, int nC, int R, int NS) {
  const int x = id % kXcds, slot = id / kXcds, nP = nC / R;
  const int groups = (B * H + kXcds - 1) / kXcds;
  const int bh = head_on_xcd(slot / nP, x, groups, line_heads(NS));
  return ChunkId{slot % nP, bh % H, bh / H, bh < B * H};
}
__device__ __forceinline__ ChunkId chunk_id(const ChunkArgs& p, bool by_cost, bool late_first) {
  return decode_chunk(blockIdx.x, p.B, p.H, p.nC, p.NS, by_cost, late_first);
}
__host__ __device__ inline int64_t chunk_grid_size(int B, int H, int nC) {
  return (int64_t)nC * ((B * H + kXcds - 1) / kXcds) * kXcds;
}
inline dim3 chunk_grid(const ChunkArgs& p) { return dim3((unsigned)chunk_grid_size(p.B, p.H, p.nC)); }
// kPair: the same decode over the nC / R runs of a head (c = run index)
__device__ __forceinline__ ChunkId run_id(const ChunkArgs& p) { return decode_run(blockIdx.x, p.B, p.H, p.nC, p.R, p.NS); }
__host__ __device__ inline int64_t run_grid_size(int B, int H, int nC, int R) {
  return (int64_t)(nC / R) * ((B * H + kXcds - 1) / kXcds) * kXcds;
}
inline dim3 run_grid(const ChunkArgs& p) { return dim3((unsigned)run_grid_size(p.B, p.H, p.nC, p.R)); }

// Backward workspace slot (in units of one Dh x N state) of the adjoint
// leaving run `run` (R chunks) of head bh = b * H + h: each head holds
// ceil(nC / R) slots.  The adjoint scan and the aggregate / state-pass
// kernels write these slots, the pipelined and pair chunk kernels read them,
// and rr_ssd_workspace_extent bounds them on the host.
__host__ __device__ inline int64_t adj_slot(int64_t bh, int nC, int R, int run) {
  return bh * ((nC + R - 1) / R) + run;
}
// Backward dA partial slot (N floats) of run `run` of head bh, nR runs per
// head: each backward workgroup writes one (the whole-head mode one run per
// head, the pair mode nC / R, the per-chunk modes nC).
__host__ __device__ inline int64_t dA_slot(int64_t bh, int nR, int run) { return bh * nR + run; }

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
//                 a zero start (into checkpoint slot k);
//       backward: G_k = (gam o dY_k)^T C_k, the adjoint the chunk sends back to
//                 its start (into the workspace).
//  2. pass_kernel, one thread per state element, walks the chunks in order:
//       forward:  h_k = tot_k h_{k-1} + S_k   (h_{-1} = h0), into slot k
//       backward: lam_k = adjoint of the state leaving chunk k,
//                 lam_{nC-1} = dfinal, lam_{k-1} = tot_k lam_k + G_k,
//                 and dh0 = tot_0 lam_0 + G_0.
//  3. the main kernel, one workgroup per chunk, reads its entering state
//     (and, backward, lam_k) and does the chunk's dense products.
// agg_kernel: a workgroup of four waves per chunk; wave w forms the 16x16
// blocks w NBW .. w NBW + NBW - 1 of the aggregate (one row block of the state
// for Dh = 64).  The operands are read with k = step: U (forward) and the
// N-wide B / C are staged in LDS in their natural [step][column] layout and
// read back by transposing reads; the backward's fp32 dY goes straight into
// A-operand registers (lane (j, g) = (lane % 16, lane / 16): dY[8 g + e][16 db
// + j]), is weighted by gam and split into bf16 hi + lo there.  The forward's
// factor m31 w is applied to the B fragments in registers.
constexpr int kAggThreads = 256;
template <int DH, int NS, bool GLA>
struct AggSmem {
  static constexpr int PX = DH + 16, PY = NS == 16 ? 16 : NS + 16;   // see DirectSmem
  uint16_t X[Q][PX];    // kind 0: U [s][d]
  uint16_t Y[Q][PY];    // B [s][n] (kind 0) or C [t][n] (kind 1)
  float wsh[Q];         // kind 0: m31_s w_s; kind 1: gam_t
};
template <int DH, int NS, bool GLA>
__global__ __launch_bounds__(kAggThreads) void agg_kernel(ChunkArgs p, int kind) {
  using S = AggSmem<DH, NS, GLA>;
  constexpr int NBN = NS / 16, NB = (DH / 16) * NBN, NBW = (NB + 3) / 4;
  constexpr int NDB = NBW > NBN ? NBW / NBN : 1;   // row blocks per wave
  __shared__ __attribute__((aligned(16))) S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int jl = lane & 15, gl = lane >> 4;
  const ChunkId id = chunk_id(p, false, false);
  if (!id.valid) return;
  const int c = id.c, h = id.h, b = id.b;
  const float a = head_rate<GLA>(p, h);
  const int64_t rowH = p.H, row0 = (int64_t)b * p.L + (int64_t)c * Q;
  constexpr int T = kAggThreads;
  constexpr int UV = (Q * DH / 8 + T - 1) / T, BV = (Q * NS / 8 + T - 1) / T;
  const int jw0 = w * NBW;                       // this wave's first block
  const bool busy = jw0 < NB;
  const int db0 = busy ? jw0 / NBN : 0;          // its first row block
  // loads first
  u16x8_t uv[UV], bv[BV];
  float dyv[NDB][8];
  if (kind == 0) {
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + T * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
      uv[v] = i < Q * DH / 8 ? *reinterpret_cast<const u16x8_t*>(p.u + ((row0 + tl) * rowH + h) * DH + d0) : u16x8_t{};
    }
  } else {
#pragma unroll
    for (int q = 0; q < NDB; ++q)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        dyv[q][e] = p.dy[((row0 + 8 * gl + e) * rowH + h) * DH + 16 * min(db0 + q, DH / 16 - 1) + jl];
  }
  const uint16_t* bsrc = kind == 0 ? p.Bm : p.Cm;
#pragma unroll
  for (int v = 0; v < BV; ++v) {
    const int i = tid + T * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
    bv[v] = i < Q * NS / 8 ? *reinterpret_cast<const u16x8_t*>(bsrc + ((row0 + tl) * rowH + h) * NS + n0) : u16x8_t{};
  }
  if (w == 0) {
    float xl = bf_val(p.delta[(row0 + (lane & (Q - 1))) * rowH + h]);   // unconditional load
    rr::pin(xl);
    const float xv = lane < Q ? xl : (GLA ? 1.f : 0.f);
    const StepScalars sc = step_scalars<GLA>(xv, a, lane);
    if (lane < Q) sm.wsh[lane] = kind == 0 ? sc.m31 * sc.w : sc.gam;
    if (lane == 0) p.tot[((int64_t)b * p.H + h) * p.nC + c] = sc.tot;
  }
  if (kind == 0) {
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + T * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
      if (i < Q * DH / 8) *reinterpret_cast<u16x8_t*>(&sm.X[tl][d0]) = uv[v];
    }
  }
#pragma unroll
  for (int v = 0; v < BV; ++v) {
    const int i = tid + T * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
    if (i < Q * NS / 8) *reinterpret_cast<u16x8_t*>(&sm.Y[tl][n0]) = bv[v];
  }
  __syncthreads();
  if (!busy) return;
  // this lane's step factors (steps 8 g .. 8 g + 7; broadcast reads)
  const float4 c0 = *reinterpret_cast<const float4*>(&sm.wsh[8 * gl]);
  const float4 c1 = *reinterpret_cast<const float4*>(&sm.wsh[8 * gl + 4]);
  const float cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  float* dst = kind == 0 ? p.ckpt + (((int64_t)b * p.H + h) * p.nC + c) * DH * NS
                          : p.agg + adj_slot((int64_t)b * p.H + h, p.nC, 1, c) * DH * NS;
#pragma unroll
  for (int q = 0; q < NDB; ++q) {
    const int db = db0 + q;
    if (db * NBN >= NB || db * NBN >= jw0 + NBW) break;
    u16x8_t xh, xl;   // A operand (rows d, k = step): U (kind 0: hi only) or gam o dY hi, lo
    if (kind == 0) {
      xh = frag_tr(&sm.X[0][16 * db], S::PX, lane);
    } else {
      float xw[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) xw[e] = cw[e] * dyv[q][e];
      rr::bf_split8(xw, xh, xl);
    }
#pragma unroll
    for (int nb = 0; nb < NBN; ++nb) {
      const int j = db * NBN + nb;
      if (j < jw0 || j >= jw0 + NBW) continue;
      const u16x8_t yr = frag_tr(&sm.Y[0][16 * nb], S::PY, lane);   // B operand (k = step, columns n)
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      if (kind == 0) {
        float yw[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) yw[e] = cw[e] * bf_val(yr[e]);
        u16x8_t yh, yl;
        rr::bf_split8(yw, yh, yl);
        acc = mfma16(xh, yh, acc);
        acc = mfma16(xh, yl, acc);
      } else {
        acc = mfma16(xh, yr, acc);
        acc = mfma16(xl, yr, acc);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) dst[(16 * db + 4 * gl + r) * NS + 16 * nb + jl] = acc[r];
    }
  }
}

// Sequential pass over the chunks of one (batch, head), one state element per
// thread.  The loads of kPass chunks go out together, unconditionally (chunk
// indices clamped into range; out-of-range terms are dropped in the fold), so
// that no branch waits on a load.
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
        const int k = min(k0 + q, nC - 1);
        sv[q] = buf[(int64_t)k * DH * NS];
        tv[q] = tot[k];
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
    float* buf = p.agg + adj_slot(bh, nC, 1, 0) * (DH * NS) + e;
    float x = p.dfinal != nullptr ? p.dfinal[bh * DH * NS + es] : 0.f;
    for (int k0 = nC - 1; k0 >= 0; k0 -= kPass) {
      float gv[kPass], tv[kPass];
#pragma unroll
      for (int q = 0; q < kPass; ++q) {
        const int k = max(k0 - q, 0);
        gv[q] = buf[(int64_t)k * DH * NS];
        tv[q] = tot[k];
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

// ------------------------------------------------------------------ state scan
// The state of the pipelined mode: one workgroup per (batch, head) walks the
// chunks in order (the backward from the last chunk), carrying the state
// (forward) or adjoint (backward) in registers and writing it once per chunk:
//   forward:  h_k = tot_k h_{k-1} + U_k^T diag(m31 o w) B_k (h_{-1} = h0),
//             into checkpoint slot k;
//   backward: slot k of the workspace <- lam_k (lam_{nC-1} = dfinal),
//             lam_{k-1} = tot_k lam_k + (gam o dY_k)^T C_k, dh0 = lam_{-1};
//             with R > 1 (kPair) only lam_k of every R-th chunk, into slot k / R.
// A chunk's update is a rank-32 MFMA product on the running state.  All 256
// threads load the chunk's inputs kScanPF chunks ahead and stage them in a
// double-buffered LDS area in natural [step][column] layout (the fp32 factor
// applied and split into bf16 hi + lo on the way: forward on B, backward on
// dY); the operands are read back by transposing LDS reads (k = step); one
// workgroup barrier per chunk.  Wave w owns the 16x16 state blocks w, w + 4,
// ...  Its traffic is the inputs it reads and the states it writes, nothing
// else (no per-chunk aggregates in HBM).
constexpr int kScanPF = 4;
template <int DH, int NS, bool BWD>
struct ScanSmem {
  static constexpr int PX = DH + 16, PY = NS == 16 ? 16 : NS + 16;   // see DirectSmem
  uint16_t X[2][BWD ? 2 : 1][Q][PX];   // fwd: U; bwd: (gam o dY) hi, lo   [step][d]
  uint16_t Y[2][BWD ? 1 : 2][Q][PY];   // fwd: (m31 w o B) hi, lo; bwd: C   [step][n]
};
template <int DH, int NS, bool GLA, bool BWD>
__global__ __launch_bounds__(256) void scan_kernel(ChunkArgs p) {
  using S = ScanSmem<DH, NS, BWD>;
  constexpr int NBN = NS / 16, NB = (DH / 16) * NBN, NBW = (NB + 3) / 4;
  constexpr int XN = BWD ? Q * DH / 4 : Q * DH / 8;   // X pieces per chunk (float4 of dY / u16x8 of U)
  constexpr int YN = Q * NS / 8;                      // Y pieces (u16x8 of B / C)
  constexpr int XV = (XN + 255) / 256, YV = (YN + 255) / 256;
  __shared__ __attribute__((aligned(16))) S sm;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l15 = lane & 15, l4 = lane >> 4;
  const int h = blockIdx.x, b = blockIdx.y;
  const int64_t bh = (int64_t)b * p.H + h, rowH = p.H;
  const float a = head_rate<GLA>(p, h);
  const int nC = p.nC;
  const float neutral = GLA ? 1.f : 0.f;

  // the running state, this wave's blocks in the [d][n] accumulator layout
  f32x4_t st[NBW];
  {
    const float* ext = BWD ? p.dfinal : p.h0;
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int j = w + 4 * i, db = j / NBN, nb = j % NBN;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        st[i][r] = j < NB && ext != nullptr
                       ? ext[bh * DH * NS + state_off<GLA, DH, NS>(16 * db + 4 * l4 + r, 16 * nb + l15)]
                       : 0.f;
    }
  }
  // chunk of walk position k (clamped: the surplus prefetches repeat the last)
  auto chunk_at = [&](int k) {
    k = min(k, nC - 1);
    return BWD ? nC - 1 - k : k;
  };
  u16x8_t xu[kScanPF][BWD ? 1 : XV], yv[kScanPF][YV];
  float4 xf[kScanPF][BWD ? XV : 1];
  float xs[kScanPF];
  auto load = [&](int slot, int k) {
    const int64_t row0 = (int64_t)b * p.L + (int64_t)chunk_at(k) * Q;
    xs[slot] = bf_val(p.delta[(row0 + (lane & (Q - 1))) * rowH + h]);   // lanes >= 32 masked at use
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int i = min(tid + 256 * v, XN - 1);   // in range (surplus threads repeat a piece)
      if constexpr (BWD) {
        const int t = i / (DH / 4), d0 = 4 * (i % (DH / 4));
        xf[slot][v] = *reinterpret_cast<const float4*>(p.dy + ((row0 + t) * rowH + h) * DH + d0);
      } else {
        const int t = i / (DH / 8), d0 = 8 * (i % (DH / 8));
        xu[slot][v] = *reinterpret_cast<const u16x8_t*>(p.u + ((row0 + t) * rowH + h) * DH + d0);
      }
    }
    const uint16_t* ysrc = BWD ? p.Cm : p.Bm;
#pragma unroll
    for (int v = 0; v < YV; ++v) {
      const int i = min(tid + 256 * v, YN - 1), t = i / (NS / 8), n0 = 8 * (i % (NS / 8));
      yv[slot][v] = *reinterpret_cast<const u16x8_t*>(ysrc + ((row0 + t) * rowH + h) * NS + n0);
    }
  };
#pragma unroll
  for (int q = 0; q < kScanPF; ++q) load(q, q);

  // this head's slots: nC checkpoints (forward), or one adjoint per run of
  // R chunks (backward; the workspace holds ceil(nC / R) per head)
  float* out = BWD ? p.agg + adj_slot(bh, nC, p.R, 0) * DH * NS : p.ckpt + bh * nC * DH * NS;
  auto store_state = [&](float* dst) {
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int j = w + 4 * i, db = j / NBN, nb = j % NBN;
      if (NB % 4 == 0 || j < NB) {
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[(16 * db + 4 * l4 + r) * NS + 16 * nb + l15] = st[i][r];
      }
    }
  };
  // Stage walk position k from prefetch slot q (a compile-time index) into
  // LDS buffer k & 1, the factor applied on the way, then refill slot q with
  // position k + kScanPF; returns tot_k.
  auto stage = [&](int k, auto qc) {
    constexpr int q = decltype(qc)::value;
    const int buf = k & 1;
    // step scalars (every wave; lanes s and s + 32 hold step s)
    const StepScalars sc = step_scalars<GLA>(lane < Q ? xs[q] : neutral, a, lane);
    const float cf = BWD ? sc.gam : sc.m31 * sc.w;
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int i = tid + 256 * v;
      if constexpr (BWD) {
        const int t = (i / (DH / 4)) & (Q - 1), d0 = 4 * (i % (DH / 4));
        const float ct = __shfl(cf, t);   // every lane (the shuffle reads other lanes)
        if (i < XN) {
          const float4 g = xf[q][v];
          u16x4_t hi, lo;
          rr::bf_split4(f32x4_t{ct * g.x, ct * g.y, ct * g.z, ct * g.w}, hi, lo);
          *reinterpret_cast<u16x4_t*>(&sm.X[buf][0][t][d0]) = hi;
          *reinterpret_cast<u16x4_t*>(&sm.X[buf][BWD ? 1 : 0][t][d0]) = lo;
        }
      } else {
        const int t = i / (DH / 8), d0 = 8 * (i % (DH / 8));
        if (i < XN) *reinterpret_cast<u16x8_t*>(&sm.X[buf][0][t][d0]) = xu[q][v];
      }
    }
#pragma unroll
    for (int v = 0; v < YV; ++v) {
      const int i = tid + 256 * v, t = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
      if constexpr (BWD) {
        if (i < YN) *reinterpret_cast<u16x8_t*>(&sm.Y[buf][0][t][n0]) = yv[q][v];
      } else {
        const float ct = __shfl(cf, t);
        if (i < YN) {
          float yw[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) yw[e] = ct * bf_val(yv[q][v][e]);
          u16x8_t hi, lo;
          rr::bf_split8(yw, hi, lo);
          *reinterpret_cast<u16x8_t*>(&sm.Y[buf][0][t][n0]) = hi;
          *reinterpret_cast<u16x8_t*>(&sm.Y[buf][BWD ? 0 : 1][t][n0]) = lo;
        }
      }
    }
    load(q, k + kScanPF);   // this slot's registers are free
    return sc.tot;
  };
  // The update of walk position k from LDS buffer k & 1: state = tot_k state + X^T Y.
  auto update = [&](int k, float tot) {
    const int buf = k & 1;
    const int c = chunk_at(k);
    if constexpr (BWD) {   // lam_c, the adjoint leaving chunk c (every R-th chunk: uniform branch, no loads)
      if (p.R == 1) store_state(out + (int64_t)c * DH * NS);
      else if (c % p.R == p.R - 1) store_state(out + (int64_t)(c / p.R) * DH * NS);
    }
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int j = w + 4 * i, db = j / NBN, nb = j % NBN;
      if (NB % 4 == 0 || j < NB) {
        f32x4_t acc = st[i] * tot;
        if constexpr (BWD) {
          const u16x8_t yr = frag_tr(&sm.Y[buf][0][0][16 * nb], S::PY, lane);
          acc = mfma16(frag_tr(&sm.X[buf][0][0][16 * db], S::PX, lane), yr, acc);
          acc = mfma16(frag_tr(&sm.X[buf][BWD ? 1 : 0][0][16 * db], S::PX, lane), yr, acc);
        } else {
          const u16x8_t xa = frag_tr(&sm.X[buf][0][0][16 * db], S::PX, lane);
          acc = mfma16(xa, frag_tr(&sm.Y[buf][0][0][16 * nb], S::PY, lane), acc);
          acc = mfma16(xa, frag_tr(&sm.Y[buf][BWD ? 0 : 1][0][16 * nb], S::PY, lane), acc);
        }
        st[i] = acc;
      }
    }
    if constexpr (!BWD) store_state(out + (int64_t)c * DH * NS);   // h_c, the state leaving chunk c
  };
  // Software pipeline: position k + 1 is staged (into the other LDS buffer)
  // while position k's update runs, one barrier per position.  In groups of
  // kScanPF positions with no exit inside (the waits for a slot's loads then
  // stay exact), then the remainder; staging past the last position repeats
  // the last chunk into a buffer nobody reads.
  static_assert(kScanPF == 4, "the walk below is unrolled by four");
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  float tot_next = stage(0, I0{});
  __syncthreads();
  const int nMain = nC - nC % kScanPF;
  for (int k0 = 0; k0 < nMain; k0 += kScanPF) {
    float tot = tot_next;
    tot_next = stage(k0 + 1, I1{});
    update(k0 + 0, tot);
    __syncthreads();
    tot = tot_next;
    tot_next = stage(k0 + 2, I2{});
    update(k0 + 1, tot);
    __syncthreads();
    tot = tot_next;
    tot_next = stage(k0 + 3, I3{});
    update(k0 + 2, tot);
    __syncthreads();
    tot = tot_next;
    tot_next = stage(k0 + 4, I0{});
    update(k0 + 3, tot);
    __syncthreads();
  }
  if (nMain + 0 < nC) {
    const float tot = tot_next;
    tot_next = stage(nMain + 1, I1{});
    update(nMain + 0, tot);
    __syncthreads();
  }
  if (nMain + 1 < nC) {
    const float tot = tot_next;
    tot_next = stage(nMain + 2, I2{});
    update(nMain + 1, tot);
    __syncthreads();
  }
  if (nMain + 2 < nC) {
    const float tot = tot_next;
    tot_next = stage(nMain + 3, I3{});
    update(nMain + 2, tot);
    __syncthreads();
  }
  if (BWD && p.dh0 != nullptr) {
#pragma unroll
    for (int i = 0; i < NBW; ++i) {
      const int j = w + 4 * i, db = j / NBN, nb = j % NBN;
      if (j < NB) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          p.dh0[bh * DH * NS + state_off<GLA, DH, NS>(16 * db + 4 * l4 + r, 16 * nb + l15)] = st[i][r];
      }
    }
  }
}

// The states of the pipelined mode: with enough heads to fill the GPU, the
// per-head scan (HBM traffic: inputs and states only); with few heads, whose
// serial walks would leave most CUs idle (measured at B3 H12 nC16: 14.7 µs
// against 9.5 µs), the aggregate kernel and the per-element state pass.
constexpr int64_t kScanMinHeads = 320;
template <int DH, int NS, bool GLA>
int launch_scan(const ChunkArgs& p, int64_t B, hipStream_t s, bool bwd) {
  const int kind = bwd ? 1 : 0;
  if (B * p.H < kScanMinHeads) {
    if (p.R != 1) return fail(RR_EINVAL, "chunked adjoint pass: one adjoint per chunk only");
    hipLaunchKernelGGL((agg_kernel<DH, NS, GLA>), chunk_grid(p), dim3(kAggThreads), 0, s, p, kind);
    if (int rc = check_launch(bwd ? "chunked backward aggregates" : "chunked forward aggregates")) return rc;
    hipLaunchKernelGGL((pass_kernel<DH, NS, GLA>), dim3(DH * NS / 256, p.H, (unsigned)B), dim3(256), 0, s, p, kind);
    return check_launch(bwd ? "chunked backward adjoint pass" : "chunked forward state pass");
  }
  if (bwd) hipLaunchKernelGGL((scan_kernel<DH, NS, GLA, true>), dim3(p.H, (unsigned)B), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((scan_kernel<DH, NS, GLA, false>), dim3(p.H, (unsigned)B), dim3(256), 0, s, p);
  return check_launch(bwd ? "chunked backward adjoint scan" : "chunked forward state scan");
}

// ------------------------------------------------------------------ direct mode
// Short sequences (nC <= kDirectMaxChunks): one workgroup per chunk forms the
// state entering its chunk (forward) or the adjoint leaving it (backward)
// itself, as a weighted sum over the raw inputs of all earlier (later)
// chunks, so a pass is a single kernel with no aggregate or state-pass kernels:
//   forward:  h_in(c) = Gam h0 + sum_{j<c} U_j^T diag(F_j m31 o w) B_j,
//             F_j = tot_{j+1} ... tot_{c-1},   Gam = tot_0 ... tot_{c-1};
//   backward: lam(c) = Gam dfinal + sum_{j>c} (F_j gam o dY_j)^T C_j,
//             F_j = tot_{c+1} ... tot_{j-1},   Gam = tot_{c+1} ... tot_{nC-1}
// (m31, w, gam and tot of chunk j as in step_scalars).  Wave w takes chunks
// j0 + w, j0 + w + 4, ... of the range (at most kDirectPerWave).  Their inputs
// are loaded up to four chunks ahead.  The bf16 operands are staged in the
// wave's own LDS area in their natural [step][column] layout (forward: B
// with the fp32 factor applied, split into bf16 hi + lo) and read back as
// MFMA operands (k = step) by transposing LDS reads; the backward's fp32 dY
// is loaded straight into its operand layout (each lane eight steps of one
// column) and weighted and split in registers, which keeps it out of LDS.
// No transposed copies and no workgroup barriers in the loop.  Each wave
// accumulates every 16x16 block of the state; the four partial sums are added
// in a fixed order (deterministic).
constexpr int kDirectMaxChunks = 16;
constexpr int kDirectMaxState = 64 * 64;   // Dh * N (the partial sums live in LDS)
constexpr int kDirectPerWave = kDirectMaxChunks / 4;

template <int DH, int NS, bool BWD>
struct alignas(16) DirectSmem {
  // a 64 x 64 state's staging areas packed, so that three workgroups fit a CU
  using SX = Staged<DH, DH * NS >= 4096>;
  using SY = Staged<NS, DH * NS >= 4096>;
  union {
    struct {   // every member 16-byte aligned (16-byte and transposing LDS accesses)
      alignas(16) uint16_t X[BWD ? 8 : SX::SIZE];      // fwd: U [s][d] (the backward's dY stays in registers)
      alignas(16) uint16_t Y[BWD ? 1 : 2][SY::SIZE];   // fwd: (F m31 w o B) hi, lo [s][n]; bwd: C [t][n]
      alignas(16) float cw[BWD ? Q : 4];               // bwd: the chunk's step factors F gam_t
    } st[4];
    float red[2][DH * NS];              // partial sums of waves 0 + 2 and 1 + 3, [d][n]
    // DH = 64 (row-owned reduction; backward with NS = 16): wave w's
    // partials of the row blocks db != w (slot db - (db > w)), 16x16 blocks
    // as [lane][4]
    float xch[DH == 64 && (!BWD || NS == 16) ? 4 : 1][3][NS / 16][256];
  };
  float tot[kDirectMaxChunks];          // decays of the chunks of the range
  float g0[BWD ? DH * NS : 1];          // backward, chunk 0's own term G_0 (see direct_sum)
};

struct NoLoads {
  __device__ void operator()() const {}
};

// Runs the weighted sum; afterwards red[] holds the two partial sums and the
// return value is Gam.  Every thread of the (256-thread) workgroup must call
// it.  `pre` is called once per thread when its wave has staged its last
// chunk: the caller issues its own chunk's loads there, so that they land
// while the partial sums are added, without their registers being live in
// the loop.  G0 (backward): the workgroup of chunk 0 also forms the
// initial-state gradient dh0 = tot_0 lam(0) + G_0, G_0 = (gam o dY_0)^T C_0,
// by taking chunk 0 into its range with a separate accumulator, and stores it
// (when dh0 is given).
template <int DH, int NS, bool GLA, bool BWD, bool G0 = false, typename PRE = NoLoads>
__device__ float direct_sum(const ChunkArgs& p, int c, int b, int h, float a, DirectSmem<DH, NS, BWD>& s,
                            float* dh0 = nullptr, PRE pre = PRE{}, f32x4_t* own = nullptr) {
  using S = DirectSmem<DH, NS, BWD>;
  constexpr int NBD = DH / 16, NBN = NS / 16;
  // DH = 64, forward or backward with NS = 16: row-owned.  Wave w ends up
  // with the full sum of row block db = w in `own` (one exchange through LDS,
  // one barrier; red[] is not used).  The forward accumulates its blocks
  // transposed (element r at n = 16 nb + 4 (lane / 16) + r, d = 16 db +
  // lane % 16: the layout of its state registers); the backward's are in the
  // natural layout (d = 16 db + 4 (lane / 16) + r, n = 16 nb + lane % 16),
  // that of its adjoint registers.
  constexpr bool ROWS = DH == 64 && (!BWD || NS == 16);
  constexpr int XV = Q * DH / 8 / 64;                           // fwd, per lane and chunk: u16x8 of U
  constexpr int YV = Q * NS / 8 / 64;                           // u16x8 of B (fwd) or C (bwd)
  constexpr int VPC = BWD ? 8 * NBD + 4 * YV : 4 * (XV + YV);   // registers per chunk in flight
  // budget for them (GLA's 64 x 64 forward: one chunk, its accumulators
  // taking 64 of the 168 registers that three workgroups per CU leave)
  constexpr int REGS = GLA && !BWD && DH * NS >= 4096 ? VPC : BWD && NS > 16 ? 48 : 80;
  constexpr int PF = REGS / VPC >= 4 ? 4 : REGS / VPC >= 2 ? 2 : 1;   // chunks in flight per wave
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t rowH = p.H;
  const bool g0 = G0 && BWD && c == 0 && dh0 != nullptr;
  const int kfirst = BWD ? c + 1 : 0;          // first chunk whose decay enters the factors
  const int j0 = g0 ? 0 : kfirst;
  const int j1 = BWD ? p.nC : c;               // the range: chunks [j0, j1)
  const int cnt = j1 - j0;
  const int nw = cnt > w ? (cnt - w + 3) / 4 : 0;   // this wave's chunks (uniform per wave)
  const float neutral = GLA ? 1.f : 0.f;
  // chunk k of this wave, clamped into the range (with an empty range, this
  // workgroup's own chunk).  Every wave issues the loads of kDirectPerWave
  // chunks whatever its count nw, so that every path has the same loads in
  // flight and the waits for a slot stay exact; a surplus chunk's loads
  // (k >= nw, never read) take one address in every lane (`on` = 0 drops the
  // lane's part of the offset): one cache line per load instead of a chunk's
  // worth of L2 traffic in the start-up burst of every workgroup.
  auto chunk = [&](int k) { return cnt > 0 ? min(j0 + w + 4 * k, j1 - 1) : c; };

  // 1. step inputs of this wave's chunks, then the operands of the first PF
  float xs[kDirectPerWave];
#pragma unroll
  for (int k = 0; k < kDirectPerWave; ++k) {
    const int64_t row0 = (int64_t)b * p.L + (int64_t)chunk(k) * Q;
    const int tl = k < nw ? lane & (Q - 1) : 0;
    xs[k] = bf_val(p.delta[(row0 + tl) * rowH + h]);   // lanes >= 32 masked below
  }
  // forward: U rows as 16-byte pieces; backward: dY in the A-operand layout
  // of 16x16x32, lane (j, g) = (lane % 16, lane / 16) holding dY[8 g + e][16 db + j]
  u16x8_t xu[PF][BWD ? 1 : XV], yv[PF][YV];
  float xg[PF][BWD ? NBD : 1][BWD ? 8 : 1];
  const int jl = lane & 15, gl = lane >> 4;
  auto load = [&](int slot, int k) {
    const int64_t row0 = (int64_t)b * p.L + (int64_t)chunk(k) * Q;
    const int on = k < nw ? 1 : 0;   // wave-uniform
    if constexpr (BWD) {
      const int64_t lo = on * ((int64_t)8 * gl * rowH * DH + jl);
#pragma unroll
      for (int db = 0; db < NBD; ++db)
#pragma unroll
        for (int e = 0; e < 8; ++e) xg[slot][db][e] = p.dy[((row0 + e) * rowH + h) * DH + 16 * db + lo];
    } else {
#pragma unroll
      for (int v = 0; v < XV; ++v) {
        const int i = on * (lane + 64 * v), t = i / (DH / 8), d0 = 8 * (i % (DH / 8));
        xu[slot][v] = *reinterpret_cast<const u16x8_t*>(p.u + ((row0 + t) * rowH + h) * DH + d0);
      }
    }
    const uint16_t* ysrc = BWD ? p.Cm : p.Bm;
#pragma unroll
    for (int v = 0; v < YV; ++v) {
      const int i = on * (lane + 64 * v), t = i / (NS / 8), n0 = 8 * (i % (NS / 8));
      yv[slot][v] = *reinterpret_cast<const u16x8_t*>(ysrc + ((row0 + t) * rowH + h) * NS + n0);
    }
  };
#pragma unroll
  for (int k = 0; k < PF; ++k) load(k, k);
#pragma unroll
  for (int k = 0; k < kDirectPerWave; ++k) rr::pin(xs[k]);   // waits for the step inputs only

  // 2. step scalars; the chunk decays go to LDS
  float coef[kDirectPerWave];
#pragma unroll
  for (int k = 0; k < kDirectPerWave; ++k) {
    const StepScalars sc = step_scalars<GLA>(lane < Q ? xs[k] : neutral, a, lane);
    coef[k] = BWD ? sc.gam : sc.m31 * sc.w;
    if (k < nw && lane == 0) s.tot[chunk(k) - j0] = sc.tot;
  }
  __syncthreads();

  // 3. chunk factors by a product scan over the range (lane i: chunk j0 + i)
  //    fwd: F_j = tot_{j+1} ... tot_{j1-1} (exclusive suffix product);
  //    bwd: F_j = tot_{kfirst} ... tot_{j-1} (exclusive prefix product; with
  //    chunk 0 in the range for dh0, tot_0 is left out)
  float gam_all;
  float fk[kDirectPerWave];
  {
    const int i = lane & 31;
    float v;
    if constexpr (BWD) {
      const int src = i - 1;   // exclusive: lane i takes chunk j0 + i - 1
      const float t = s.tot[min(max(src, 0), kDirectMaxChunks - 1)];   // read in every lane
      v = src >= 0 && src < cnt && j0 + src >= kfirst ? t : 1.f;
    } else {
      const int src = cnt - i;   // reversed, exclusive: lane i takes chunk j0 + cnt - i
      const float t = s.tot[min(max(src, 0), kDirectMaxChunks - 1)];   // read in every lane
      v = i > 0 && src >= 0 && src < cnt ? t : 1.f;
    }
    const float e = prefix_prod32(v, lane);   // lane i: product over lanes 0 .. i
    gam_all = __shfl(e, min(cnt, 31));
#pragma unroll
    for (int k = 0; k < kDirectPerWave; ++k) {
      const int idx = chunk(k) - j0;
      fk[k] = __shfl(e, BWD ? idx : cnt - 1 - idx);
    }
  }

  // 4. this wave's chunks: stage, then accumulate every block of the state
  f32x4_t acc[NBD][NBN];
#pragma unroll
  for (int db = 0; db < NBD; ++db)
#pragma unroll
    for (int nb = 0; nb < NBN; ++nb) acc[db][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto& st = s.st[w];
#pragma unroll
  for (int k = 0; k < kDirectPerWave; ++k) {
    if (k >= nw) break;
    const int slot = k % PF;
    const float cf = coef[k] * fk[k];   // lane s < 32: the factor of step s
    if constexpr (BWD) {
      if (lane < Q) st.cw[lane] = cf;
#pragma unroll
      for (int v = 0; v < YV; ++v) {
        const int i = lane + 64 * v, t = i / (NS / 8), n0 = 8 * (i % (NS / 8));
        *reinterpret_cast<u16x8_t*>(&st.Y[0][S::SY::off(t, n0)]) = yv[slot][v];
      }
      wave_lds_sync();
      // this lane's step factors (steps 8 g .. 8 g + 7; broadcast reads)
      const float4 c0 = *reinterpret_cast<const float4*>(&st.cw[8 * gl]);
      const float4 c1 = *reinterpret_cast<const float4*>(&st.cw[8 * gl + 4]);
      const float cwl[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      u16x8_t yf[NBN];
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) yf[nb] = frag_tr_st<typename S::SY>(st.Y[0], 16 * nb, lane);
#pragma unroll
      for (int db = 0; db < NBD; ++db) {
        float xw[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) xw[e] = cwl[e] * xg[slot][db][e];
        u16x8_t xh, xl;
        rr::bf_split8(xw, xh, xl);
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          acc[db][nb] = mfma16(xh, yf[nb], acc[db][nb]);
          acc[db][nb] = mfma16(xl, yf[nb], acc[db][nb]);
        }
      }
      // the registers of this slot are free: the loads of chunk k + PF
      // (issued even past this wave's last chunk, as single-address surplus
      // loads, so that the waits for a slot stay exact)
      if (k + PF < kDirectPerWave) load(slot, k + PF);
    } else {
#pragma unroll
      for (int v = 0; v < XV; ++v) {
        const int i = lane + 64 * v, t = i / (DH / 8), d0 = 8 * (i % (DH / 8));
        *reinterpret_cast<u16x8_t*>(&st.X[S::SX::off(t, d0)]) = xu[slot][v];
      }
#pragma unroll
      for (int v = 0; v < YV; ++v) {
        const int i = lane + 64 * v, t = i / (NS / 8), n0 = 8 * (i % (NS / 8));
        const float ct = __shfl(cf, t);
        float yw[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) yw[e] = ct * bf_val(yv[slot][v][e]);
        u16x8_t hi, lo;
        rr::bf_split8(yw, hi, lo);
        *reinterpret_cast<u16x8_t*>(&st.Y[0][S::SY::off(t, n0)]) = hi;
        *reinterpret_cast<u16x8_t*>(&st.Y[BWD ? 0 : 1][S::SY::off(t, n0)]) = lo;
      }
      // the registers of this slot are free: the loads of chunk k + PF (see above)
      if (k + PF < kDirectPerWave) load(slot, k + PF);
      wave_lds_sync();
      u16x8_t yf[2][NBN];
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
        for (int hl = 0; hl < 2; ++hl) yf[hl][nb] = frag_tr_st<typename S::SY>(st.Y[hl], 16 * nb, lane);
#pragma unroll
      for (int db = 0; db < NBD; ++db) {
        const u16x8_t xfr = frag_tr_st<typename S::SX>(st.X, 16 * db, lane);
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          if constexpr (ROWS) {   // transposed block: (B^T U)[n][d]
            acc[db][nb] = mfma16(yf[0][nb], xfr, acc[db][nb]);
            acc[db][nb] = mfma16(yf[1][nb], xfr, acc[db][nb]);
          } else {
            acc[db][nb] = mfma16(xfr, yf[0][nb], acc[db][nb]);
            acc[db][nb] = mfma16(xfr, yf[1][nb], acc[db][nb]);
          }
        }
      }
    }
    if constexpr (G0) {
      if (g0 && w == 0 && k == 0) {   // chunk 0: its own term, set aside in LDS
        const int l15 = lane & 15, l4 = lane >> 4;
#pragma unroll
        for (int db = 0; db < NBD; ++db)
#pragma unroll
          for (int nb = 0; nb < NBN; ++nb) {
#pragma unroll
            for (int r = 0; r < 4; ++r) s.g0[(16 * db + 4 * l4 + r) * NS + 16 * nb + l15] = acc[db][nb][r];
            acc[db][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
          }
      }
    }
    wave_lds_sync();   // the next chunk's staging rewrites the area
  }
  pre();

  if constexpr (ROWS) {
    // 5. row-owned: wave w hands its partials of the other row blocks over,
    // then sums row block w over the four waves in a fixed order
    __syncthreads();   // the staging areas are dead (xch[] overlays them)
    f32x4_t mine[NBN];
#pragma unroll
    for (int db = 0; db < NBD; ++db) {
      if (db == w) {
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) mine[nb] = acc[db][nb];
      } else {
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb)
          *reinterpret_cast<f32x4_t*>(&s.xch[w][db - (db > w ? 1 : 0)][nb][4 * lane]) = acc[db][nb];
      }
    }
    __syncthreads();
#pragma unroll
    for (int nb = 0; nb < NBN; ++nb) own[nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int src = 0; src < 4; ++src) {
      const int slot = min(w - (w > src ? 1 : 0), 2);   // in bounds; unused for src == w
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) {
        const f32x4_t v = *reinterpret_cast<const f32x4_t*>(&s.xch[src][slot][nb][4 * lane]);
        own[nb] += src == w ? mine[nb] : v;
      }
    }
    if constexpr (G0) {
      if (g0) {
        // dh0 = tot_0 lam(0) + G_0 for this wave's rows (natural layout)
        const int l15 = lane & 15, l4 = lane >> 4;
        const float t0 = s.tot[0];
        const float* ext = p.dfinal != nullptr ? p.dfinal + ((int64_t)b * p.H + h) * DH * NS : nullptr;
        float* out = dh0 + ((int64_t)b * p.H + h) * DH * NS;
        f32x4_t lam[NBN];
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) lam[nb] = own[nb];
        if (ext != nullptr) {
#pragma unroll
          for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              lam[nb][r] += gam_all * ext[state_off<GLA, DH, NS>(16 * w + 4 * l4 + r, 16 * nb + l15)];
        }
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int d = 16 * w + 4 * l4 + r, n = 16 * nb + l15;
            out[state_off<GLA, DH, NS>(d, n)] = t0 * lam[nb][r] + s.g0[d * NS + n];
          }
      }
    }
    return gam_all;
  }

  // 5. partial sums: red[0] = acc_0 + acc_2, red[1] = acc_1 + acc_3
  __syncthreads();   // the staging areas are dead (red[] overlays them)
  const int l15 = lane & 15, l4 = lane >> 4;
  auto at = [&](int db, int nb, int r) { return (16 * db + 4 * l4 + r) * NS + 16 * nb + l15; };
  if (w >= 2) {
#pragma unroll
    for (int db = 0; db < NBD; ++db)
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) s.red[w - 2][at(db, nb, r)] = acc[db][nb][r];
  }
  __syncthreads();
  if (w < 2) {
#pragma unroll
    for (int db = 0; db < NBD; ++db)
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int e = at(db, nb, r);
          s.red[w][e] = acc[db][nb][r] + s.red[w][e];
        }
  }
  __syncthreads();
  if constexpr (G0) {
    if (g0) {
      // dh0 = tot_0 lam(0) + G_0, lam(0) = red0 + red1 + Gam dfinal; every
      // thread takes elements e = tid + 256 k (the LDS reads first, the
      // dfinal terms in one branch)
      constexpr int PER = DH * NS / 256;
      const float t0 = s.tot[0];
      const float* ext = p.dfinal != nullptr ? p.dfinal + ((int64_t)b * p.H + h) * DH * NS : nullptr;
      float* out = dh0 + ((int64_t)b * p.H + h) * DH * NS;
      float lam[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int e = tid + 256 * k;
        lam[k] = s.red[0][e] + s.red[1][e];
      }
      if (ext != nullptr) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
          const int e = tid + 256 * k;
          lam[k] += gam_all * ext[state_off<GLA, DH, NS>(e / NS, e % NS)];
        }
      }
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int e = tid + 256 * k;
        out[state_off<GLA, DH, NS>(e / NS, e % NS)] = t0 * lam[k] + s.g0[e];
      }
    }
  }
  return gam_all;
}

// Element (d, n) of the direct sum is direct_partial (the two partials in
// red[]) plus, where the caller has an h0 (forward) or dfinal (backward),
// direct_ext (Gam times that element).  Callers read all their partials
// first and add the ext terms in one separate branch: a branch per element
// would wait for each LDS read before the next is issued.
template <int DH, int NS, bool BWD>
__device__ __forceinline__ float direct_partial(const DirectSmem<DH, NS, BWD>& s, int d, int n) {
  const int e = d * NS + n;
  return s.red[0][e] + s.red[1][e];
}
template <int DH, int NS, bool GLA>
__device__ __forceinline__ float direct_ext(float gam_all, const float* ext, int d, int n) {
  return gam_all * ext[state_off<GLA, DH, NS>(d, n)];
}

// ------------------------------------------------------------------ direct mode, wide states
// The same sums for states past kDirectMaxState (Dh 128 with N 64, GLA's
// 128 x 128), whose every-block accumulators would not fit one wave's
// registers and whose partial sums would not fit the LDS: every wave walks
// every summed chunk and accumulates only the state blocks its kernel owns,
// in that kernel's register layout, so nothing is reduced across waves:
//   forward (fwd_kernel): row blocks db = w + 4 i, every column block nb,
//     transposed (element r at n = 16 nb + 4 (lane / 16) + r, d = 16 db +
//     lane % 16): acc[i][nb] += ((F m31 w) o B)^T U;
//   backward (col_bwd_kernel): column blocks nb = w + 4 i, every row block
//     db, natural (element r at d = 16 db + 4 (lane / 16) + r, n = 16 nb +
//     lane % 16): acc[i][db] += ((F gam) o dY)^T C.
// A summed chunk is staged once per workgroup: each thread loads its pieces
// (the loads of the chunk two ahead are in flight meanwhile), applies the fp32
// step factors to the fp32-weighted operand (forward B, backward dY) and
// splits it into bf16 hi + lo; then every wave reads its operands by
// transposing LDS reads (16x16x32 MFMA, two per block and chunk).  The step
// scalars of the range (wave w: chunks j0 + w + 4 k) and the chunk factors F_j
// are formed first, as in direct_sum.  With g0 (backward, chunk 0) chunk 0's
// step scalars are formed as well (range index 0), for the caller's dh0.
// (Measured against it at Dh 128, B3 L512 H12: weighting U instead of B,
// row-owned backward sums redistributed through memory, and double-buffered
// staging overlapping the products were each no faster.  Probes that drop
// one part of the loop each — the products, the barriers, the weighting and
// splitting, the L2 misses — save at most a third of the sum's time: it is
// the dependent latency of each summed chunk.)
template <int DH, int NS, bool BWD>
struct alignas(16) WideSmem {
  using SX = Staged<DH>;   // fwd: U [s][d]; bwd: (F gam o dY) hi, lo [t][d]
  using SY = Staged<NS>;   // fwd: (F m31 w o B) hi, lo [s][n]; bwd: C [t][n]
  uint16_t X[BWD ? 2 : 1][SX::SIZE];
  uint16_t Y[BWD ? 1 : 2][SY::SIZE];
  float coef[kDirectMaxChunks][Q];   // step factors of the range's chunks: m31 w (fwd), gam (bwd)
  float tot[kDirectMaxChunks];       // their chunk decays gam_31
};

template <int DH, int NS, bool GLA, bool BWD, int NI, int NJ>
__device__ float direct_sum_wide(const ChunkArgs& p, int c, int b, int h, float a, WideSmem<DH, NS, BWD>& s,
                                 f32x4_t (&acc)[NI][NJ], bool g0) {
  using S = WideSmem<DH, NS, BWD>;
  using SX = typename S::SX;
  using SY = typename S::SY;
  constexpr int NBD = DH / 16, NBN = NS / 16;
  static_assert(NJ == (BWD ? NBD : NBN) && NI == (BWD ? (NBN + 3) / 4 : (NBD + 3) / 4), "direct_sum_wide: blocks");
  static_assert(DH % 64 == 0 && NS % 64 == 0, "direct_sum_wide: whole pieces per thread");
  // pieces per thread and chunk: fwd U rows (8 bf16), bwd dY rows (4 fp32); B / C rows (8 bf16)
  constexpr int XV = BWD ? Q * DH / 4 / 256 : Q * DH / 8 / 256, XW = BWD ? DH / 4 : DH / 8;
  constexpr int YV = Q * NS / 8 / 256;
  using XT = std::conditional_t<BWD, float4, u16x8_t>;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t rowH = p.H;
  const int kfirst = BWD ? c + 1 : 0;          // first summed chunk
  const int j0 = BWD && g0 ? 0 : kfirst;       // range with step scalars: [j0, j1)
  const int j1 = BWD ? p.nC : c;
  const int cnt = j1 - j0;
  const int ns = j1 - kfirst;                  // summed chunks: [kfirst, j1)
  const int nw = cnt > w ? (cnt - w + 3) / 4 : 0;   // this wave's chunks of the range (uniform per wave)
  const float neutral = GLA ? 1.f : 0.f;
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // 1. step scalars of the range's chunks into LDS
  {
    auto chunk = [&](int k) { return cnt > 0 ? min(j0 + w + 4 * k, j1 - 1) : c; };
    float xs[kDirectPerWave];
#pragma unroll
    for (int k = 0; k < kDirectPerWave; ++k) {
      const int64_t row0 = (int64_t)b * p.L + (int64_t)chunk(k) * Q;
      const int tl = k < nw ? lane & (Q - 1) : 0;
      xs[k] = bf_val(p.delta[(row0 + tl) * rowH + h]);   // lanes >= 32 take the neutral input below
    }
#pragma unroll
    for (int k = 0; k < kDirectPerWave; ++k) {
      if (k < nw) {
        const StepScalars sc = step_scalars<GLA>(lane < Q ? xs[k] : neutral, a, lane);
        const int jj = chunk(k) - j0;
        if (lane < Q) s.coef[jj][lane] = BWD ? sc.gam : sc.m31 * sc.w;
        if (lane == 0) s.tot[jj] = sc.tot;
      }
    }
  }
  __syncthreads();

  // 2. chunk factors by a product scan over the range (lane i: range index
  //    i), in every wave: fwd F_j = tot_{j+1} ... tot_{j1-1} at lane
  //    cnt - 1 - i, bwd F_j = tot_{kfirst} ... tot_{j-1} at lane i
  float e;
  {
    const int i = lane & 31;
    float v;
    if constexpr (BWD) {
      const int src = i - 1;
      const float t = s.tot[min(max(src, 0), kDirectMaxChunks - 1)];   // read in every lane
      v = src >= 0 && src < cnt && j0 + src >= kfirst ? t : 1.f;
    } else {
      const int src = cnt - i;
      const float t = s.tot[min(max(src, 0), kDirectMaxChunks - 1)];   // read in every lane
      v = i > 0 && src >= 0 && src < cnt ? t : 1.f;
    }
    e = prefix_prod32(v, lane);
  }
  const float gam_all = __shfl(e, min(cnt, 31));
  if (ns <= 0) return gam_all;   // workgroup-uniform

  // 3. the summed chunks, two slots of loads in flight.  Summed chunk k is
  //    chunk kfirst + k; past the last one (k >= ns) the loads repeat one
  //    address of the last chunk in every lane and its factor is 0 (the
  //    weighted operand is staged as zeros and the products add 0), so every
  //    pass of the loop runs the same loads, waits and products.
  XT xr[2][XV];
  u16x8_t yr[2][YV];
  auto load = [&](int slot, int k) {
    const int on = k < ns ? 1 : 0;   // uniform
    const int64_t row0 = (int64_t)b * p.L + (int64_t)(kfirst + min(k, ns - 1)) * Q;
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int i = on * (tid + 256 * v), t = i / XW, x0 = (BWD ? 4 : 8) * (i % XW);
      if constexpr (BWD)
        xr[slot][v] = *reinterpret_cast<const float4*>(p.dy + ((row0 + t) * rowH + h) * DH + x0);
      else
        xr[slot][v] = *reinterpret_cast<const u16x8_t*>(p.u + ((row0 + t) * rowH + h) * DH + x0);
    }
    const uint16_t* ysrc = BWD ? p.Cm : p.Bm;
#pragma unroll
    for (int v = 0; v < YV; ++v) {
      const int i = on * (tid + 256 * v), t = i / (NS / 8), n0 = 8 * (i % (NS / 8));
      yr[slot][v] = *reinterpret_cast<const u16x8_t*>(ysrc + ((row0 + t) * rowH + h) * NS + n0);
    }
  };
  auto stage = [&](int slot, int k) {
    const bool live = k < ns;                      // uniform
    const int jj = kfirst + min(k, ns - 1) - j0;   // range index
    const float F = __shfl(e, BWD ? jj : cnt - 1 - jj);
#pragma unroll
    for (int v = 0; v < XV; ++v) {
      const int i = tid + 256 * v, t = i / XW, x0 = (BWD ? 4 : 8) * (i % XW);
      if constexpr (BWD) {
        const float cf = live ? F * s.coef[jj][t] : 0.f;
        const float4 g = xr[slot][v];
        u16x4_t hi, lo;
        rr::bf_split4(f32x4_t{cf * g.x, cf * g.y, cf * g.z, cf * g.w}, hi, lo);
        *reinterpret_cast<u16x4_t*>(&s.X[0][SX::off(t, x0)]) = hi;
        *reinterpret_cast<u16x4_t*>(&s.X[BWD ? 1 : 0][SX::off(t, x0)]) = lo;
      } else {
        *reinterpret_cast<u16x8_t*>(&s.X[0][SX::off(t, x0)]) = xr[slot][v];
      }
    }
#pragma unroll
    for (int v = 0; v < YV; ++v) {
      const int i = tid + 256 * v, t = i / (NS / 8), n0 = 8 * (i % (NS / 8));
      if constexpr (BWD) {
        *reinterpret_cast<u16x8_t*>(&s.Y[0][SY::off(t, n0)]) = yr[slot][v];
      } else {
        const float cf = live ? F * s.coef[jj][t] : 0.f;
        float yw[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) yw[q] = cf * bf_val(yr[slot][v][q]);
        u16x8_t hi, lo;
        rr::bf_split8(yw, hi, lo);
        *reinterpret_cast<u16x8_t*>(&s.Y[0][SY::off(t, n0)]) = hi;
        *reinterpret_cast<u16x8_t*>(&s.Y[BWD ? 0 : 1][SY::off(t, n0)]) = lo;
      }
    }
  };
  auto products = [&]() {
    if constexpr (BWD) {
      u16x8_t cf[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) cf[i] = frag_tr_st<SY>(s.Y[0], 16 * min(w + 4 * i, NBN - 1), lane);
#pragma unroll
      for (int db = 0; db < NBD; ++db) {
        const u16x8_t xh = frag_tr_st<SX>(s.X[0], 16 * db, lane);
        const u16x8_t xl = frag_tr_st<SX>(s.X[BWD ? 1 : 0], 16 * db, lane);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          if (w + 4 * i < NBN) {
            acc[i][db] = mfma16(xh, cf[i], acc[i][db]);
            acc[i][db] = mfma16(xl, cf[i], acc[i][db]);
          }
        }
      }
    } else {
      u16x8_t xf[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) xf[i] = frag_tr_st<SX>(s.X[0], 16 * min(w + 4 * i, NBD - 1), lane);
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) {
        const u16x8_t yh = frag_tr_st<SY>(s.Y[0], 16 * nb, lane);
        const u16x8_t yl = frag_tr_st<SY>(s.Y[BWD ? 0 : 1], 16 * nb, lane);
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          if (w + 4 * i < NBD) {
            acc[i][nb] = mfma16(yh, xf[i], acc[i][nb]);
            acc[i][nb] = mfma16(yl, xf[i], acc[i][nb]);
          }
        }
      }
    }
  };
  load(0, 0);
  load(1, 1);
  for (int k = 0; k < ns; k += 2) {
    stage(0, k);
    load(0, k + 2);
    __syncthreads();
    products();
    __syncthreads();
    stage(1, k + 1);   // past the last summed chunk: zeros
    load(1, k + 3);
    __syncthreads();
    products();
    __syncthreads();
  }
  return gam_all;
}

// ------------------------------------------------------------------ forward
// TRB (SSD with N <= 32): the end state reads B transposed from LDS and
// weights it in registers; otherwise (m31 o w o B)^T is staged as BwT.
template <int DH, int NS, bool TRB>
struct alignas(16) FwdSmem {
  uint16_t Ut[DH][PQ];                                     // U^T  [d][s]
  uint16_t C[Q][Cfg<DH, NS>::PN];                          // C    [t][n]
  uint16_t B[Q][TRB ? Staged<NS>::P : Cfg<DH, NS>::PN];    // B    [s][n]
  uint16_t BwT_hi[TRB ? 1 : NS][PQ];                       // (m31 o w o B)^T [n][s]
  uint16_t BwT_lo[TRB ? 1 : NS][PQ];
  uint16_t W_hi[Q][PQ];                                    // M o CB^T o w_s  [t][s]
  uint16_t W_lo[Q][PQ];
  float x[Q];       // step input (SSD delta, GLA gate)
  float cd[4][Q];   // SSD: cumulative delta (a copy per wave)
  float gam[Q];
  float wend[Q];    // TRB: m31 o w, the step factors of the end state
};

template <int DH, int NS, bool DIRECT, bool TRB>
union FwdShared {
  FwdSmem<DH, NS, TRB> f;
};
// The direct sums' LDS: the narrow form's (DirectSmem) up to kDirectMaxState,
// the wide form's (WideSmem) past it.
template <int DH, int NS, bool BWD>
using DirectLds = std::conditional_t<(DH * NS <= kDirectMaxState), DirectSmem<DH, NS, BWD>, WideSmem<DH, NS, BWD>>;
template <int DH, int NS, bool TRB>
union FwdShared<DH, NS, true, TRB> {
  FwdSmem<DH, NS, TRB> f;
  DirectLds<DH, NS, false> d;
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
// GLA's direct mode, and the wide direct mode: three workgroups per CU where
// the LDS allows it (a chunk per workgroup, so every workgroup of a 16-chunk
// sequence at batch 3 can be resident); the register budget follows.
template <int DH, int NS, int MODE, bool GLA>
constexpr int kFwdWgs = (GLA || DH * NS > kDirectMaxState) && MODE == kDirect &&
                                160 * 1024 / sizeof(FwdShared<DH, NS, true, !GLA && NS <= 32>) >= 3
                            ? 3
                            : 1;

template <int DH, int NS, int MODE, bool GLA>
__global__ __launch_bounds__(256, (kFwdWgs<DH, NS, MODE, GLA>)) void fwd_kernel(ChunkArgs p) {
  constexpr int NBD = DH / 16, NBN = NS / 16;
  constexpr int DBW = (NBD + 3) / 4;   // row blocks per wave
  constexpr bool STATE = MODE == kWhole || MODE == kDirect;   // forms the chunk's end state
  constexpr bool TRB = !GLA && NS <= 32;
  __shared__ FwdShared<DH, NS, MODE == kDirect, TRB> smu;
  auto& sm = smu.f;
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l15 = lane & 15, l4 = lane >> 4;
  int h, b, cbeg;
  if constexpr (MODE == kWhole) {
    h = blockIdx.y, b = blockIdx.z, cbeg = 0;
  } else {
    const ChunkId id = chunk_id(p, MODE == kDirect, MODE == kDirect);   // late chunks cost most
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
  // the chunk's own inputs (all loads issued before any use)
  constexpr int UV = (Q * DH / 8 + 255) / 256, BV = (Q * NS / 8 + 255) / 256;
  u16x8_t uv[UV], bv[BV], cv[BV];
  float xv;
  // (direct mode, where the loads are issued during the sum and consumed
  // after it: every load unconditional and in bounds, threads past the
  // chunk's pieces repeating one (the LDS writes below skip them), since a
  // load under a branch makes the branch's join wait for all loads in flight;
  // the other modes consume them at once and skip the surplus loads)
  auto issue = [&](int c, int tid) {
    const int64_t row0 = (int64_t)b * p.L + (int64_t)c * Q;
#pragma unroll
    for (int v = 0; v < UV; ++v) {
      const int i = tid + 256 * v, tl = (i / (DH / 8)) & (Q - 1), d0 = 8 * (i % (DH / 8));
      uv[v] = MODE == kDirect || i < Q * DH / 8
                  ? *reinterpret_cast<const u16x8_t*>(p.u + ((row0 + tl) * rowH + h) * DH + d0)
                  : u16x8_t{};
    }
#pragma unroll
    for (int v = 0; v < BV; ++v) {
      const int i = tid + 256 * v, tl = (i / (NS / 8)) & (Q - 1), n0 = 8 * (i % (NS / 8));
      const int64_t g = ((row0 + tl) * rowH + h) * NS + n0;
      const bool ld = MODE == kDirect || i < Q * NS / 8;
      bv[v] = ld ? *reinterpret_cast<const u16x8_t*>(p.Bm + g) : u16x8_t{};
      cv[v] = ld ? *reinterpret_cast<const u16x8_t*>(p.Cm + g) : u16x8_t{};
    }
    // unconditional (in-bounds) load, so no branch waits on it
    xv = bf_val(p.delta[(row0 + (tid & (Q - 1))) * rowH + h]);
  };
  if constexpr (MODE == kDirect && DH * NS > kDirectMaxState) {
    // wide state: every wave sums its own rows of the state (direct_sum_wide),
    // then the chunk's loads go out
    const float gam_all = direct_sum_wide<DH, NS, GLA, false>(p, cbeg, b, h, a, smu.d, hst, false);
    issue(cbeg, tid);
    if (p.h0 != nullptr) {
      const float* h0b = p.h0 + bh * DH * NS;
#pragma unroll
      for (int i = 0; i < DBW; ++i) {
        const int db = w + 4 * i;
        if (db < NBD) {
#pragma unroll
          for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              hst[i][nb][r] += direct_ext<DH, NS, GLA>(gam_all, h0b, 16 * db + l15, 16 * nb + 4 * l4 + r);
        }
      }
    }
    __syncthreads();   // the chunk below reuses the LDS of the sum
  } else if constexpr (MODE == kDirect) {
    // the chunk's loads go out when each wave has staged its last summed chunk
    f32x4_t own[DH == 64 ? NBN : 1];
    const float gam_all =
        direct_sum<DH, NS, GLA, false>(p, cbeg, b, h, a, smu.d, nullptr, [&] { issue(cbeg, tid); }, own);
    const float* h0b = p.h0 != nullptr ? p.h0 + bh * DH * NS : nullptr;
    if constexpr (DH == 64) {   // row block w, summed in registers
#pragma unroll
      for (int nb = 0; nb < NBN; ++nb) hst[0][nb] = own[nb];
    } else {
#pragma unroll
      for (int i = 0; i < DBW; ++i) {
        const int db = w + 4 * i;
        if (db < NBD) {
#pragma unroll
          for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) hst[i][nb][r] = direct_partial(smu.d, 16 * db + l15, 16 * nb + 4 * l4 + r);
        }
      }
    }
    if (h0b != nullptr) {
#pragma unroll
      for (int i = 0; i < DBW; ++i) {
        const int db = w + 4 * i;
        if (db < NBD) {
#pragma unroll
          for (int nb = 0; nb < NBN; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
              hst[i][nb][r] += direct_ext<DH, NS, GLA>(gam_all, h0b, 16 * db + l15, 16 * nb + 4 * l4 + r);
        }
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

  // whole head with a 64-column state: the next chunk's loads are issued as
  // soon as this chunk's are staged (the first before the loop; the last
  // chunk repeats itself, so the count of loads in flight is the same every
  // time).  Measured on one box: GLA B96 L512 H12 forward 161 -> 152 us; SSD
  // config 4 (N = 128) 1110 -> 1127 us, so not there; N = 16 (SSD B96)
  // 95 -> 108 us.
  constexpr bool PREF = MODE == kWhole && NS == 64;
  if constexpr (PREF) issue(cbeg, tid);
  for (int c = cbeg; c < cend; ++c) {
    // a fresh copy of the thread index per chunk keeps the compiler from
    // hoisting every per-lane address of the body out of the chunk loop
    int tidv = tid;
    if constexpr (MODE == kWhole) asm volatile("" : "+v"(tidv));
    const int tid = tidv, lane = tidv & 63, l15 = lane & 15, l4 = lane >> 4;
    const int64_t row0 = (int64_t)b * p.L + (int64_t)c * Q;  // first (b, t) row of the chunk
    // ---- stage the chunk's inputs
    {
      if constexpr (MODE != kDirect && !PREF) issue(c, tid);
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
      if constexpr (PREF) issue(min(c + 1, cend - 1), tid);
    }
    __syncthreads();
    // ---- step scalars (every wave; lanes s and s + 32 hold step s), then
    // W = M o C B^T o w_s and, unless TRB, (m31 o w o B)^T.  SSD: W's rows
    // split over the waves (t = 8 w + 4 (lane / 32) + q, the r32row rows
    // r = 4 w + q), BwT over all threads.  GLA: wave 0 forms W while the
    // others stage BwT (measured: the split's redundant C B^T products and
    // decay chains cost GLA more than they save).
    const StepScalars sc = step_scalars<GLA>(sm.x[lane & (Q - 1)], a, lane);
    if (lane < Q) {
      if constexpr (!GLA) sm.cd[w][lane] = sc.cd;   // this wave's copy, for its decays
      if (w == 0) {
        sm.gam[lane] = sc.gam;
        if constexpr (TRB) sm.wend[lane] = sc.m31 * sc.w;
      }
    }
    auto stage_bwt = [&](int first, int stride) {
      // lane s (and s + 32) weights column s
      const float wend = sc.m31 * sc.w;
      for (int i = first; i < Q * NS; i += stride) {
        const int n = i / Q, s2 = i % Q;
        uint16_t hi, lo;
        bf_split(wend * bf_val(sm.B[s2][n]), hi, lo);
        sm.BwT_hi[n][s2] = hi;
        sm.BwT_lo[n][s2] = lo;
      }
    };
    if constexpr (GLA) {
      if (w == 0) {
        f32x16_t cb = {};
#pragma unroll
        for (int kb = 0; kb < NS / 16; ++kb)
          cb = mfma32(frag(&sm.C[lane & 31][16 * kb + 8 * (lane >> 5)]),
                      frag(&sm.B[lane & 31][16 * kb + 8 * (lane >> 5)]), cb);
        const int s = lane & 31;
        float m[16];
        decay_block32<true>(sm.x, a, lane, m);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int t = r32row(r, lane);
          uint16_t hi, lo;
          bf_split(m[r] * sc.w * cb[r], hi, lo);
          sm.W_hi[t][s] = hi;
          sm.W_lo[t][s] = lo;
        }
      } else if constexpr (STATE) {
        stage_bwt(tid - 64, 192);
      }
    } else {
      wave_lds_sync();   // this wave's cd
      f32x16_t cb = {};   // C B^T, every wave (its rows picked below)
#pragma unroll
      for (int kb = 0; kb < NS / 16; ++kb)
        cb = mfma32(frag(&sm.C[lane & 31][16 * kb + 8 * (lane >> 5)]),
                    frag(&sm.B[lane & 31][16 * kb + 8 * (lane >> 5)]), cb);
      float cq[4];
      switch (w) {   // uniform
        case 0: cq[0] = cb[0], cq[1] = cb[1], cq[2] = cb[2], cq[3] = cb[3]; break;
        case 1: cq[0] = cb[4], cq[1] = cb[5], cq[2] = cb[6], cq[3] = cb[7]; break;
        case 2: cq[0] = cb[8], cq[1] = cb[9], cq[2] = cb[10], cq[3] = cb[11]; break;
        default: cq[0] = cb[12], cq[1] = cb[13], cq[2] = cb[14], cq[3] = cb[15]; break;
      }
      const int s = lane & 31, t0 = 8 * w + 4 * (lane >> 5);
      const float cds = sm.cd[w][s];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float mq = masked_exp(s <= t0 + q, a * (sm.cd[w][t0 + q] - cds));   // M[t0 + q][s]
        uint16_t hi, lo;
        bf_split(mq * sc.w * cq[q], hi, lo);
        sm.W_hi[t0 + q][s] = hi;
        sm.W_lo[t0 + q][s] = lo;
      }
      if constexpr (STATE && !TRB) stage_bwt(tid, 256);
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
        // TRB: the (m31 o w o B)^T operands from B's k-runs (transposing LDS
        // reads), weighted per step and split in registers (steps
        // s = 8 (lane / 16) + e); else from BwT
        float wl[8];
        if constexpr (TRB) {
          const float4 w0 = *reinterpret_cast<const float4*>(&sm.wend[8 * l4]);
          const float4 w1 = *reinterpret_cast<const float4*>(&sm.wend[8 * l4 + 4]);
          wl[0] = w0.x, wl[1] = w0.y, wl[2] = w0.z, wl[3] = w0.w, wl[4] = w1.x, wl[5] = w1.y, wl[6] = w1.z, wl[7] = w1.w;
        }
#pragma unroll
        for (int nb = 0; nb < NBN; ++nb) {
          u16x8_t bh, bl;
          if constexpr (TRB) {
            const u16x8_t braw = frag_tr(&sm.B[0][16 * nb], Staged<NS>::P, lane);
            float bw[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) bw[e] = wl[e] * bf_val(braw[e]);
            rr::bf_split8(bw, bh, bl);
          } else {
            bh = frag(&sm.BwT_hi[16 * nb + l15][8 * l4]);
            bl = frag(&sm.BwT_lo[16 * nb + l15][8 * l4]);
          }
          f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
          acc = mfma16(bh, fu, acc);
          acc = mfma16(bl, fu, acc);
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
    if (int rc = launch_scan<DH, NS, GLA>(p, B, s, false)) return rc;
    hipLaunchKernelGGL((fwd_kernel<DH, NS, kPipe, GLA>), chunk_grid(p), dim3(256), 0, s, p);
  } else if (p.mode == kDirect || p.mode == kSum) {   // R == 1; kSum forward = direct
    // (wide: the states the host picks it for, SSD Dh 128 with N 64 and GLA Dh 128)
    if constexpr (DH * NS <= kDirectMaxState || (DH % 64 == 0 && NS % 64 == 0 && (GLA || (DH == 128 && NS == 64))))
      hipLaunchKernelGGL((fwd_kernel<DH, NS, kDirect, GLA>), chunk_grid(p), dim3(256), 0, s, p);
    else
      return fail(RR_EUNSUPPORTED, "chunked forward: no direct mode for this state");
  } else {   // R == nC
    hipLaunchKernelGGL((fwd_kernel<DH, NS, kWhole, GLA>), dim3(1, p.H, (unsigned)B), dim3(256), 0, s, p);
  }
  return check_launch("chunked forward");
}

}  // namespace chunked
}  // namespace rr
