// rr_tiles.h — tiled chained scan for the bandwidth-bound diagonal
// recurrences (RG-LRU, rotLRU): packed vector loads and the cross-tile
// state hand-off.
//
// A pass is one kernel over tiles of (channels x steps).  A tile loads its
// inputs once into registers, folds them into the tile's affine map, receives
// the state entering the tile from its predecessor, hands its own exit state
// to its successor, and replays its steps from registers.  The hand-off:
//   - tiles take tickets from an atomic counter in the caller's workspace and
//     map tickets to tiles so that every predecessor of a tile holds a smaller
//     ticket; a tile only ever waits for a workgroup that already runs (or has
//     finished), so the waits always end;
//   - a state value travels as one 64-bit word (float bits | tag << 32)
//     written and read with agent-scope atomics: the word validates itself,
//     so no cache-flushing fence is needed, and the chain is deterministic
//     (each tile waits for exactly its predecessor);
//   - the spin is bounded (kMaxSpin) so the kernel terminates whatever
//     happens, and tickets beyond the tile count end their workgroup at once;
//     a wait that expires sets a bit in the library's device status word
//     (read by rr_async_status) and hands on NaN, so the pass's results are
//     visibly invalid instead of silently wrong;
//   - the workspace is cleared by clear_kernel before each pass, and a pass
//     also leaves it clear: a consumer zeroes the slot it has read and the
//     holder of the last ticket zeroes the counter (so a pass replayed
//     without the clear, e.g. an isolated graph node, still runs correctly).
#pragma once

#include <algorithm>

#include "rr_common.h"

namespace rr {
namespace tiles {

constexpr uint32_t kTag = 1;           // "published in this pass"
constexpr int kMaxSpin = 1 << 20;      // bounded wait (about a second): never reached in practice
constexpr int kWsHeader = 64;          // u32 words before the hand-off slots (counter at [0])
constexpr uint32_t kStatusSpinExpired = 1;   // bit of the device status word (rr_async_status)

// ---------------------------------------------------------------- schedule
// Tickets map to tiles so that a tile's predecessor (the tile of the same
// channels one step tile earlier, or later in a reverse-time pass) always
// holds a smaller ticket: tickets run over the nGrp channel groups fastest and
// over the K step tiles slowest.  A workgroup takes its ticket only once it
// runs, so every workgroup it waits for has started and, by induction over
// the tickets, finishes: no wait depends on a workgroup that is not resident.
struct TileOfTicket {
  int k;     // step tile
  int grp;   // channel group (batch row * G + channel tile)
};
__host__ __device__ inline TileOfTicket tile_of_ticket(int ticket, int nGrp, int K, bool reverse_time) {
  const int slow = ticket / nGrp;
  return TileOfTicket{reverse_time ? K - 1 - slow : slow, ticket % nGrp};
}

// Checkpoint interval start of the backward: the steps t0 .. of a wave resume
// from the checkpoint written after step tb - 1, tb = t0 - t0 % T (row
// tb / T - 1 of the batch row's nC checkpoints), or from the initial state
// when tb = 0.  Waves wholly past L (padding of the last step tile) read
// nothing.  Returns the checkpoint row, or -1 when no checkpoint is read.
__host__ __device__ inline int bwd_ckpt_row(int t0, int T, int L) {
  if (t0 >= L) return -1;
  const int tb = t0 - t0 % T;
  return tb > 0 ? tb / T - 1 : -1;
}

// ---------------------------------------------------------------- packed loads
// N consecutive elements of an input, kept packed in registers.
template <typename InT, int N> struct Pack;
template <> struct Pack<bf16, 4> {
  uint2 v;
  __device__ float operator[](int i) const {
    const uint32_t w = i < 2 ? v.x : v.y;
    return __uint_as_float((i & 1) ? (w & 0xffff0000u) : (w << 16));
  }
};
template <> struct Pack<bf16, 2> {
  uint32_t v;
  __device__ float operator[](int i) const { return __uint_as_float(i ? (v & 0xffff0000u) : (v << 16)); }
};
template <> struct Pack<f16, 4> {
  uint2 v;
  __device__ float operator[](int i) const {
    const uint32_t w = i < 2 ? v.x : v.y;
    const uint16_t h = (i & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
};
template <> struct Pack<f16, 2> {
  uint32_t v;
  __device__ float operator[](int i) const {
    const uint16_t h = i ? (uint16_t)(v >> 16) : (uint16_t)(v & 0xffffu);
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
};
template <> struct Pack<float, 4> {
  float4 v;
  __device__ float operator[](int i) const { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }
};
template <> struct Pack<float, 2> {
  float2 v;
  __device__ float operator[](int i) const { return i == 0 ? v.x : v.y; }
};

// fp32 -> the 16-bit input encoding (round to nearest even).
template <typename InT>
__device__ __forceinline__ uint16_t bits16(float v) {
  if constexpr (__is_same(InT, bf16)) return from_f32<bf16>(v).bits;
  else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
}

// Loads elements [i, i + N) (i a multiple of N; the tensor 16-byte aligned).
template <typename InT, int N>
__device__ __forceinline__ Pack<InT, N> ld_pack(const InT* p, int64_t i) {
  Pack<InT, N> r;
  r.v = *reinterpret_cast<const decltype(r.v)*>(p + i);
  return r;
}
// v where ok, else alt.  The loaded words are pinned first, so the load they
// come from stays unconditional (a load moved under a branch makes the
// branch's join wait for every load in flight).
template <typename InT, int N>
__device__ __forceinline__ Pack<InT, N> pick(bool ok, Pack<InT, N> v, const Pack<InT, N>& alt) {
  constexpr int W = (int)(sizeof(v.v) / 4);
  uint32_t* pv = reinterpret_cast<uint32_t*>(&v.v);
  const uint32_t* pa = reinterpret_cast<const uint32_t*>(&alt.v);
#pragma unroll
  for (int w = 0; w < W; ++w) {
    asm volatile("" : "+v"(pv[w]));
    pv[w] = ok ? pv[w] : pa[w];
  }
  return v;
}

// The identity step of a masked (out-of-range) position: value `one` everywhere.
template <typename InT, int N>
__device__ __forceinline__ Pack<InT, N> pack_fill(float one) {
  Pack<InT, N> r;
  if constexpr (sizeof(InT) == 4) {
    float* f = reinterpret_cast<float*>(&r.v);
#pragma unroll
    for (int e = 0; e < N; ++e) f[e] = one;
  } else {
    const uint16_t bits = bits16<InT>(one);
    uint16_t* h = reinterpret_cast<uint16_t*>(&r.v);
#pragma unroll
    for (int e = 0; e < N; ++e) h[e] = bits;
  }
  return r;
}

// The same accesses at a 32-bit element offset from a wave-uniform base (the
// address is then one scalar base plus one 32-bit lane offset, no 64-bit
// arithmetic per lane).
template <typename InT, int N>
__device__ __forceinline__ Pack<InT, N> ld_pack_at(const InT* base, uint32_t i) {
  Pack<InT, N> r;
  r.v = *reinterpret_cast<const decltype(r.v)*>(reinterpret_cast<const char*>(base) + i * (uint32_t)sizeof(InT));
  return r;
}

// Stores N fp32 values (16 or 8 bytes) at [i, i + N).
template <int N>
__device__ __forceinline__ void st_f32(float* p, int64_t i, const float (&v)[N]) {
  if constexpr (N == 4) *reinterpret_cast<float4*>(p + i) = make_float4(v[0], v[1], v[2], v[3]);
  else *reinterpret_cast<float2*>(p + i) = make_float2(v[0], v[1]);
}
template <int N>
__device__ __forceinline__ void st_f32_at(float* base, uint32_t i, const float (&v)[N]) {
  float* p = reinterpret_cast<float*>(reinterpret_cast<char*>(base) + i * 4u);
  if constexpr (N == 4) *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  else *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
}
// Stores N values in the input type at [i, i + N).
template <typename InT, int N>
__device__ __forceinline__ void st_pack(InT* p, int64_t i, const float (&v)[N]) {
  if constexpr (sizeof(InT) == 4) {
    st_f32<N>(reinterpret_cast<float*>(p), i, v);
  } else {
    uint16_t h[N];
#pragma unroll
    for (int e = 0; e < N; ++e) h[e] = bits16<InT>(v[e]);
    if constexpr (N == 4) *reinterpret_cast<uint2*>(p + i) = make_uint2(h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16);
    else *reinterpret_cast<uint32_t*>(p + i) = h[0] | (uint32_t)h[1] << 16;
  }
}
template <typename InT, int N>
__device__ __forceinline__ void st_pack_at(InT* base, uint32_t i, const float (&v)[N]) {
  InT* p = reinterpret_cast<InT*>(reinterpret_cast<char*>(base) + i * (uint32_t)sizeof(InT));
  st_pack<InT, N>(p, 0, v);
}

// ---------------------------------------------------------------- hand-off
__device__ __forceinline__ void publish(uint64_t* slot, float v) {
  const uint64_t word = (uint64_t)__float_as_uint(v) | ((uint64_t)kTag << 32);
  __hip_atomic_store(slot, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits (bounded) until `slot` holds a published value, clears the slot (its
// only reader is the caller) and returns the value.  If the wait expires, the
// expiry is recorded in *status and the value returned is NaN.
__device__ __forceinline__ float take_value(uint64_t* slot, uint32_t* status) {
  uint64_t word = 0;
  bool got = false;
  for (int spin = 0; spin < kMaxSpin; ++spin) {
    word = __hip_atomic_load(slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((uint32_t)(word >> 32) == kTag) {
      got = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  __hip_atomic_store(slot, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (!got) {
    __hip_atomic_fetch_or(status, kStatusSpinExpired, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __builtin_nanf("");
  }
  return __uint_as_float((uint32_t)word);
}

// Ticket of this workgroup (thread 0 takes it; every thread returns it), or
// -1 past the tile count.  The holder of the last ticket zeroes the counter:
// every other workgroup of the pass has taken its ticket by then.
__device__ __forceinline__ int take_ticket(uint32_t* counter, int ntiles, int* lds_slot) {
  if (threadIdx.x == 0) {
    const uint32_t t = atomicAdd(counter, 1u);
    if (t == (uint32_t)ntiles - 1) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lds_slot = t < (uint32_t)ntiles ? (int)t : -1;
  }
  __syncthreads();
  return __builtin_amdgcn_readfirstlane(*lds_slot);   // uniform: tile indices and bases in scalar registers
}

// Clears the ticket counter and the hand-off slots of a pass (a template so
// that every translation unit including this header may instantiate it).
template <typename W>
__global__ void clear_kernel(W* ws, int64_t nwords32) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = i; j < nwords32 / 4; j += stride) reinterpret_cast<uint4*>(ws)[j] = make_uint4(0, 0, 0, 0);
}

inline int launch_clear(void* ws, size_t bytes, hipStream_t s) {
  const int64_t n = (int64_t)(bytes / 4);
  const int64_t blocks = std::min<int64_t>((n / 4 + 255) / 256, 1024);
  hipLaunchKernelGGL(clear_kernel<uint32_t>, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256), 0, s,
                     static_cast<uint32_t*>(ws), n);
  return check_launch("clear hand-off workspace");
}

// Workspace bytes of a pass: header + one 64-bit slot per (tile, value),
// rounded to 16 bytes.
inline size_t ws_bytes(int64_t tiles, int64_t values_per_tile) {
  return ((size_t)kWsHeader * 4 + (size_t)(tiles * values_per_tile) * 8 + 15) / 16 * 16;
}
inline uint32_t* ws_counter(void* ws) { return static_cast<uint32_t*>(ws); }
inline uint64_t* ws_slots(void* ws) {
  return reinterpret_cast<uint64_t*>(static_cast<uint32_t*>(ws) + kWsHeader);
}

// Geometry of a pass: G channel tiles per batch row, K step tiles, U steps
// per wave, NW waves per workgroup (a tile spans NW * U steps).
struct Geometry {
  int G, K, U, NW;
};

}  // namespace tiles

// Pass geometries of rglru.hip (gated: the fused-gate kernels) and
// rotlru.hip (Dp pairs), as their entry points launch them.
tiles::Geometry rglru_geometry(int64_t L, int64_t D, int dtype, int pass, bool gated);
tiles::Geometry rotlru_geometry(int64_t L, int64_t Dp);

}  // namespace rr
