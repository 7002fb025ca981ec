// resident.hip — forward of the chunked SSD / GLA form (rr_chunked.h) for
// short heads: every chunk of a head resident in one workgroup.
//
// The state's d axis (SSD channel, GLA value index j) splits into independent
// 16-column slices: h[d, :] and Y[:, d] depend only on column d of U, so a
// workgroup owns one (batch, head, slice) and needs no other workgroup.  It
// runs one wave per chunk (nC <= 16 waves):
//   1. wave c loads its chunk (U slice, B, C, step inputs), forms the step
//      scalars, the chunk aggregate S_c = U^T diag(m31 o w) B (16 x N, bf16
//      MFMA, fp32 factors split into hi + lo) into LDS, and the intra-chunk
//      matrix W = M o C B^T o w_s (32 x 32, hi + lo into LDS);
//   2. one thread per state element walks the chunks in order,
//      h_in(c + 1) = gam_31(c) h_in(c) + S_c (h_in(0) = h0), leaving each
//      chunk's entering state in LDS and writing the checkpoints;
//   3. wave c forms Y^T = U^T W^T + (h_in C^T) diag(gam) for its chunk.
// Against the per-chunk direct sums (each chunk's workgroup re-reading and
// re-multiplying the inputs of all earlier chunks) every input is read once
// and the chunk-to-chunk carry is 16 fused multiply-adds per element in LDS.
// Operand layouts are those of rr_mfma.h; U and B are staged in LDS for
// transposing reads (k = step), W is stored [t][s] with its 8-column units
// permuted by row (unit u of row t at u ^ (t % 4)) against bank conflicts.
#include "rr_chunked.h"

namespace rr {
namespace chunked {
namespace {

constexpr int kResMaxChunks = 16;
constexpr int DQ = 16;   // state columns (d) per workgroup

template <int NS>
struct alignas(16) ResWave {
  using SB = Staged<NS, true>;   // B [s][n]
  using SU = Staged<DQ>;         // U slice [s][d]
  union {
    uint16_t b[SB::SIZE];
    uint16_t w[2][Q * Q];        // W hi, lo: [t][s], units permuted
  } x;
  uint16_t u[SU::SIZE];
  float g[Q];      // SSD: cumulative delta; GLA: gate
  float wend[Q];   // m31 o w, the step weights of the chunk aggregate
  float gam[Q];
};

template <int NS>
struct alignas(16) ResSmem {
  // chunk aggregates, then entering states [d][n]; rows padded by 16 bytes
  // so the 16 rows that a 16-lane operand read takes fall in distinct banks
  float st[kResMaxChunks][DQ][NS + 4];
  float tot[kResMaxChunks];
  ResWave<NS> wv[kResMaxChunks];
};

__device__ __forceinline__ int w_off(int t, int s) { return t * Q + ((((s >> 3) ^ t) & 3) << 3) + (s & 7); }

template <int NS, bool GLA>
__global__ __launch_bounds__(64 * kResMaxChunks) void res_fwd_kernel(ChunkArgs p) {
  static_assert(sizeof(ResSmem<NS>) <= 160 * 1024, "resident forward: LDS");
  using SB = typename ResWave<NS>::SB;
  using SU = typename ResWave<NS>::SU;
  constexpr int KB = NS / 16;   // 16-wide n blocks
  __shared__ ResSmem<NS> sm;
  const int nDQ = p.DH / DQ;
  const int id = blockIdx.x, xcd = id % kXcds, k = id / kXcds;
  // a head's slices share an XCD, and so do heads whose B / C rows share lines
  const int groups = (p.B * p.H + kXcds - 1) / kXcds;
  const int dq = k % nDQ, bh = head_on_xcd(k / nDQ, xcd, groups, line_heads(NS));
  if (bh >= p.B * p.H) return;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, c = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l15 = lane & 15, l4 = lane >> 4, s32 = lane & 31, hi32 = lane >> 5;
  const float a = head_rate<GLA>(p, h);
  const int H = p.H, DH = p.DH, d0 = DQ * dq;
  const int64_t row0 = (int64_t)b * p.L + (int64_t)c * Q;   // first (b, t) row of this wave's chunk
  auto rowp = [&](int s) -> int64_t { return (row0 + s) * H + h; };
  ResWave<NS>& wv = sm.wv[c];

  // ---- 1. loads (all issued before any use), in the order of their use:
  // the step input, B and C (step scalars, decays and C B^T need nothing
  // else, so they run while U is in flight), U last
  const float xv = bf_val(p.delta[rowp(s32)]);
  u16x8_t bfr[KB], cfr[KB];   // B, C rows s = lane % 32, n = 16 kb + 8 (lane / 32) + e
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int64_t off = rowp(s32) * NS + 16 * kb + 8 * hi32;
    bfr[kb] = *reinterpret_cast<const u16x8_t*>(p.Bm + off);
    cfr[kb] = *reinterpret_cast<const u16x8_t*>(p.Cm + off);
  }
  // C^T operand of the state term: column t = 16 tb + lane % 16, n-run.
  // N = 16: loaded here with the rest (8 bytes per lane); wider: a second
  // read of the C rows loaded above for C B^T, issued only when phase 2
  // starts (from L2 then), which keeps it out of the start-up burst
  constexpr int KC = NS == 16 ? 1 : NS / 32;
  u16x8_t ctf[2][KC];
  u16x4_t ctf4[2];
  auto load_ct = [&]() {
#pragma unroll
    for (int tb = 0; tb < 2; ++tb) {
      const int64_t base = rowp(16 * tb + l15) * NS;
      if constexpr (NS == 16) {
        ctf4[tb] = *reinterpret_cast<const u16x4_t*>(p.Cm + base + 4 * l4);
      } else {
#pragma unroll
        for (int kk = 0; kk < KC; ++kk)
          ctf[tb][kk] = *reinterpret_cast<const u16x8_t*>(p.Cm + base + 32 * kk + 8 * l4);
      }
    }
  };
  if constexpr (NS == 16) load_ct();
  const u16x8_t ufr = *reinterpret_cast<const u16x8_t*>(p.u + rowp(lane >> 1) * DH + d0 + 8 * (lane & 1));

  // entering state of the carry below (one element per pass of its loop)
  float h0v[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.h0 != nullptr) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = tid + i * 64 * p.nC;
      if (e < DQ * NS) {
        const int d = e / NS, n = e % NS;
        h0v[i] = p.h0[(int64_t)bh * DH * NS + (GLA ? (int64_t)n * DH + d0 + d : (int64_t)(d0 + d) * NS + n)];
      }
    }
  }

  // ---- step scalars (lanes s and s + 32 both hold step s) and the
  // elements of W = M o C B^T o w_s (registers: they are stored over the B
  // staging once the aggregate has read it)
  const StepScalars sc = step_scalars<GLA>(xv, a, lane);
  if (lane < Q) {
    wv.g[lane] = GLA ? xv : sc.cd;
    wv.wend[lane] = sc.m31 * sc.w;
    wv.gam[lane] = sc.gam;
  }
  if (lane == 0) sm.tot[c] = sc.tot;
  float wel[16];
  {
    f32x16_t cb = {};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) cb = mfma32(cfr[kb], bfr[kb], cb);
    wave_lds_sync();   // the step scalars above, for the decays
    float m[16];
    decay_block32<GLA>(wv.g, a, lane, m);
#pragma unroll
    for (int r = 0; r < 16; ++r) wel[r] = m[r] * sc.w * cb[r];
  }
  // ---- stage U and B
  *reinterpret_cast<u16x8_t*>(&wv.u[SU::off(lane >> 1, 8 * (lane & 1))]) = ufr;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) *reinterpret_cast<u16x8_t*>(&wv.x.b[SB::off(s32, 16 * kb + 8 * hi32)]) = bfr[kb];
  wave_lds_sync();

  // ---- chunk aggregate S_c[d][n] = sum_s U[s][d] wend_s B[s][n]
  const u16x8_t uT = frag_tr_st<SU>(wv.u, 0, lane);   // A: row d = lane % 16, k = s = 8 (lane / 16) + e
  {
    float uw[8];
    const float4 w0 = *reinterpret_cast<const float4*>(&wv.wend[8 * l4]);
    const float4 w1 = *reinterpret_cast<const float4*>(&wv.wend[8 * l4 + 4]);
    const float wl[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) uw[e] = wl[e] * bf_val(uT[e]);
    u16x8_t uh, ul;
    bf_split8(uw, uh, ul);
#pragma unroll
    for (int nb = 0; nb < KB; ++nb) {
      const u16x8_t bk = frag_tr_st<SB>(wv.x.b, 16 * nb, lane);   // B: col n, k = s
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
      acc = mfma16(uh, bk, acc);
      acc = mfma16(ul, bk, acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.st[c][4 * l4 + r][16 * nb + l15] = acc[r];   // D: row d, col n
    }
  }
  // ---- W, hi and lo (over the B staging: this wave's reads are done)
  wave_lds_sync();   // the transposing reads of B above precede the W stores
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int t = r32row(r, lane);
    uint16_t whi, wlo;
    bf_split(wel[r], whi, wlo);
    wv.x.w[0][w_off(t, s32)] = whi;
    wv.x.w[1][w_off(t, s32)] = wlo;
  }
  __syncthreads();
  if constexpr (NS != 16) load_ct();

  // ---- 2. chunk-to-chunk carry, one thread per state element: all LDS
  // reads, then the chain, then the LDS writes, then the checkpoint stores,
  // with no branch between them (a store followed by a wait for loads at a
  // branch join would wait for the store as well).  Slots past nC hold
  // leftovers; their results are never stored to memory.
  {
    const int nC = p.nC;
#pragma unroll
    for (int i = 0; i < 4; ++i) {   // DQ * NS <= 1024 elements, >= 256 threads per pass
      const int e = tid + i * 64 * nC;
      if (e >= DQ * NS) break;
      const int d = e / NS, n = e % NS;
      const float hfirst = h0v[i];
      float agg[kResMaxChunks], tt[kResMaxChunks], hend[kResMaxChunks];
#pragma unroll
      for (int cc = 0; cc < kResMaxChunks; ++cc) {
        agg[cc] = sm.st[cc][d][n];
        tt[cc] = sm.tot[cc];
      }
      float hcur = hfirst;
#pragma unroll
      for (int cc = 0; cc < kResMaxChunks; ++cc) {
        const float hin = hcur;
        hcur = tt[cc] * hcur + agg[cc];
        agg[cc] = hin;
        hend[cc] = hcur;
      }
#pragma unroll
      for (int cc = 0; cc < kResMaxChunks; ++cc) sm.st[cc][d][n] = agg[cc];
      float* ck = p.ckpt + ((int64_t)bh * nC * DH + d0 + d) * NS + n;
#pragma unroll
      for (int cc = 0; cc < kResMaxChunks; ++cc)
        if (cc < nC) ck[(int64_t)cc * DH * NS] = hend[cc];
    }
  }
  __syncthreads();

  // ---- 3. Y^T[d][t] = (U^T W^T)[d][t] + gam_t (h_in C^T)[d][t]
#pragma unroll
  for (int tb = 0; tb < 2; ++tb) {
    const int t = 16 * tb + l15;
    const int wo = w_off(t, 8 * l4);
    f32x4_t yi = {0.f, 0.f, 0.f, 0.f}, ys = {0.f, 0.f, 0.f, 0.f};
    yi = mfma16(uT, *reinterpret_cast<const u16x8_t*>(&wv.x.w[0][wo]), yi);
    yi = mfma16(uT, *reinterpret_cast<const u16x8_t*>(&wv.x.w[1][wo]), yi);
    if constexpr (NS == 16) {
      const float4 hv = *reinterpret_cast<const float4*>(&sm.st[c][l15][4 * l4]);   // A: row d, k = n
      u16x4_t hh, hl;
      bf_split4(f32x4_t{hv.x, hv.y, hv.z, hv.w}, hh, hl);
      ys = mfma16k16(hh, ctf4[tb], ys);
      ys = mfma16k16(hl, ctf4[tb], ys);
    } else {
#pragma unroll
      for (int kk = 0; kk < KC; ++kk) {
        const float4 h0v = *reinterpret_cast<const float4*>(&sm.st[c][l15][32 * kk + 8 * l4]);
        const float4 h1v = *reinterpret_cast<const float4*>(&sm.st[c][l15][32 * kk + 8 * l4 + 4]);
        const float hvv[8] = {h0v.x, h0v.y, h0v.z, h0v.w, h1v.x, h1v.y, h1v.z, h1v.w};
        u16x8_t hh, hl;
        bf_split8(hvv, hh, hl);
        ys = mfma16(hh, ctf[tb][kk], ys);
        ys = mfma16(hl, ctf[tb][kk], ys);
      }
    }
    const float gt = wv.gam[t];
    float4 o;
    o.x = yi[0] + gt * ys[0];
    o.y = yi[1] + gt * ys[1];
    o.z = yi[2] + gt * ys[2];
    o.w = yi[3] + gt * ys[3];
    *reinterpret_cast<float4*>(p.y + rowp(t) * DH + d0 + 4 * l4) = o;   // D: row d = 4 (lane / 16) + r, col t
  }
}

template <int NS, bool GLA>
int launch(const ChunkArgs& p, int64_t B, hipStream_t s) {
  const int64_t groups = (B * p.H + kXcds - 1) / kXcds;
  const dim3 grid((unsigned)(groups * kXcds * (p.DH / DQ)));
  hipLaunchKernelGGL((res_fwd_kernel<NS, GLA>), grid, dim3(64 * p.nC), 0, s, p);
  return check_launch("chunked forward (resident)");
}

}  // namespace
}  // namespace chunked

bool res_fwd_supported(int64_t B, int64_t H, int64_t nC, int64_t Dh, int64_t N) {
  // (the carry covers the DQ * N state elements in at most 4 passes of the
  // workgroup's 64 nC threads: 16 nC >= N)
  return nC >= 1 && nC <= chunked::kResMaxChunks && Dh % chunked::DQ == 0 && (N == 16 || N == 32 || N == 64) &&
         16 * nC >= N && B * H * (Dh / chunked::DQ) < ((int64_t)1 << 30);
}

int res_fwd(const ChunkArgs& p, int64_t B, hipStream_t s, bool gla) {
  if (gla) {
    switch (p.NS) {
      case 32: return chunked::launch<32, true>(p, B, s);
      case 64: return chunked::launch<64, true>(p, B, s);
      default: break;
    }
  } else {
    switch (p.NS) {
      case 16: return chunked::launch<16, false>(p, B, s);
      case 32: return chunked::launch<32, false>(p, B, s);
      case 64: return chunked::launch<64, false>(p, B, s);
      default: break;
    }
  }
  return fail(RR_EUNSUPPORTED, "chunked forward (resident): unsupported N");
}

}  // namespace rr
