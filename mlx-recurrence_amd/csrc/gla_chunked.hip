// gla_chunked.hip — GLA scan on bf16 MFMA (the chunked form of rr_chunked.h).
//
// GLA (reference gla.py:78-100) is the chunked recurrence of rr_chunked.h with
// u = v, B = k, C = q, d = j (value index), n = i (key index), per-step decay
// g_t and input weight 1.  The forward runs the shared kernels of
// rr_chunked.h; the backward is the column-owned kernel of chunked_bwd.hip.
// This file holds the host-side mode choice and workspace layout.
#include "rr_chunked.h"

namespace {

template <int D>
int launch_gla_fwd(const rr::ChunkArgs& p, int64_t B, hipStream_t s) {
  return rr::chunked::launch_fwd<D, D, true>(p, B, s);
}

int64_t align64(int64_t n) { return (n + 63) / 64 * 64; }

}  // namespace

namespace rr {

bool gla2_supported(int dtype, int64_t B, int64_t L, int64_t H, int64_t seg, int64_t Dh, int pass) {
  if (dtype != RR_BF16 || chunk_len(L, seg) != chunked::Q) return false;
  if ((L / chunked::Q) * ((B * H + chunked::kXcds - 1) / chunked::kXcds * chunked::kXcds) >= ((int64_t)1 << 31))
    return false;
  return Dh == 32 || Dh == 64 || Dh == 128;
}

// The direct mode (one kernel per pass, each chunk's workgroup summing over
// the other chunks' inputs) for short heads: up to 4 chunks always; up to 16
// while every workgroup can be resident at once (three per CU on 256 CUs; a
// second round of workgroups costs more than the aggregate and state-pass
// kernels it saves).
constexpr int64_t kGlaDirectMaxChunks = 4;
constexpr int64_t kGlaDirectMaxWorkgroups = 3 * 256;
// With enough heads to fill the GPU, whole heads: the forward always (the
// state in registers from chunk to chunk: no aggregates, no state pass, no
// checkpoint re-read; B96 L512 H12: 238 -> 175 us), the backward for short
// heads (the adjoint carried likewise, no adjoint scan or workspace: 383 ->
// 365 us; long heads serialise too many chunks per workgroup).
constexpr int64_t kGlaWholeMinHeads = 512;
constexpr int64_t kGlaWholeBwdMaxChunks = 16;

int gla2_mode(int64_t B, int64_t H, int64_t nC, int64_t Dh, int pass) {
  if (B * H >= kGlaWholeMinHeads && (pass == 0 || nC <= kGlaWholeBwdMaxChunks)) return chunked::kWhole;
  if (pass == 0 && res_fwd_supported(B, H, nC, Dh, Dh)) return chunked::kRes;   // short heads, resident
  if (Dh * Dh > chunked::kDirectMaxState)   // Dh 128: the wide direct mode (direct_sum_wide) while resident
    return nC <= chunked::kDirectMaxChunks && B * H * nC <= kGlaDirectMaxWorkgroups ? chunked::kDirect
                                                                                     : chunked::kPipe;
  if (nC <= kGlaDirectMaxChunks) return chunked::kDirect;
  return nC <= chunked::kDirectMaxChunks && B * H * nC <= kGlaDirectMaxWorkgroups ? chunked::kDirect : chunked::kPipe;
}

size_t gla2_ws_bytes(int64_t B, int64_t H, int64_t nC, int64_t Dh, int pass) {
  const int mode = gla2_mode(B, H, nC, Dh, pass);
  if (mode == chunked::kDirect && Dh * Dh > chunked::kDirectMaxState)   // wide: the backward's adjoints
    return pass == 1 ? (size_t)align64(B * H * nC * Dh * Dh) * sizeof(float) : 0;
  if (mode == chunked::kDirect || mode == chunked::kWhole || mode == chunked::kRes) return 0;
  int64_t f = align64(B * H * nC);
  if (pass == 1) f += align64(B * H * nC * Dh * Dh);
  return (size_t)f * sizeof(float);
}

void gla2_carve_ws(ChunkArgs& a, void* ws, int64_t B, int pass) {
  float* f = static_cast<float*>(ws);
  a.ws = a.tot = a.agg = nullptr;
  if (a.mode == chunked::kDirect && a.DH * a.DH > chunked::kDirectMaxState) {   // wide: the backward's adjoints
    a.agg = pass == 1 ? f : nullptr;
    return;
  }
  if (a.mode == chunked::kDirect || a.mode == chunked::kWhole || a.mode == chunked::kRes) return;
  a.tot = f;
  f += align64(B * a.H * a.nC);
  a.agg = pass == 1 ? f : nullptr;
}

int gla2_fwd(const ChunkArgs& p, int64_t B, hipStream_t s) {
  if (p.mode == chunked::kRes) return res_fwd(p, B, s, true);
  switch (p.DH) {
    case 32: return launch_gla_fwd<32>(p, B, s);
    case 64: return launch_gla_fwd<64>(p, B, s);
    case 128: return launch_gla_fwd<128>(p, B, s);
    default: return fail(RR_EUNSUPPORTED, "gla chunked: unsupported Dh");
  }
}

int gla2_bwd(const ChunkArgs& p, int64_t B, hipStream_t s) { return chunked_bwd_cols(p, B, s, true); }

}  // namespace rr
