// rr_abi.hip — library-wide C entry points: ABI version, error channel and the
// shared shape rules.
#include "rr_common.h"
#include "rr_tiles.h"

#include <atomic>
#include <string>

// Error bits that kernels report after the launch has returned (an expired
// bounded wait); one copy per device.
__device__ __align__(16) uint32_t g_status_word[4];

namespace rr {

namespace {
constexpr int kMaxDevices = 64;
std::atomic<uint32_t*> g_status_ptr[kMaxDevices];
}  // namespace

uint32_t* status_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    fail(RR_EHIP, "status word: no current HIP device");
    return nullptr;
  }
  uint32_t* p = g_status_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    void* addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(g_status_word)) != hipSuccess || addr == nullptr) {
      fail(RR_EHIP, "status word: hipGetSymbolAddress failed");
      return nullptr;
    }
    p = static_cast<uint32_t*>(addr);
    g_status_ptr[dev].store(p, std::memory_order_release);
  }
  return p;
}

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(RR_EHIP, std::string(what) + ": " + hipGetErrorString(e));
  }
  return RR_OK;
}

// Same three conditions and messages as check_segment_shape in the reference
// (mlx_recurrence/_chassis.py:104-115).
int check_segment_shape(int64_t L, int64_t seg, int64_t lane_dim, const char* lane_name) {
  if (seg <= 0) return fail(RR_EINVAL, "seg must be positive, got " + std::to_string(seg));
  if (L % seg != 0) {
    return fail(RR_EINVAL, "sequence length L=" + std::to_string(L) +
                               " must be divisible by seg=" + std::to_string(seg) +
                               " (segment-checkpoint pattern tiles L into L/seg segments)");
  }
  if (lane_dim % 32 != 0) {
    return fail(RR_EINVAL, std::string(lane_name) + "=" + std::to_string(lane_dim) +
                               " must be a multiple of 32 (fused gradient reductions use "
                               "32-lane simdgroups)");
  }
  return RR_OK;
}

}  // namespace rr

extern "C" int rr_abi_version(void) { return RR_ABI_VERSION; }

extern "C" const char* rr_last_error(void) { return rr::g_last_error.c_str(); }

extern "C" int64_t rr_chunk_len(int64_t L, int64_t seg) { return rr::chunk_len(L, seg); }

extern "C" int rr_async_status(void) {
  uint32_t* p = rr::status_word();
  if (p == nullptr) return RR_EHIP;
  if (hipDeviceSynchronize() != hipSuccess) return rr::fail(RR_EHIP, "rr_async_status: hipDeviceSynchronize failed");
  uint32_t v = 0;
  if (hipMemcpy(&v, p, sizeof v, hipMemcpyDeviceToHost) != hipSuccess) {
    return rr::fail(RR_EHIP, "rr_async_status: reading the status word failed");
  }
  if (v == 0) return RR_OK;
  const uint32_t zero = 0;
  if (hipMemcpy(p, &zero, sizeof zero, hipMemcpyHostToDevice) != hipSuccess) {
    return rr::fail(RR_EHIP, "rr_async_status: clearing the status word failed");
  }
  return rr::fail(RR_EHIP, "a tile hand-off wait of an RG-LRU / rotLRU pass expired (status bits " +
                               std::to_string(v) + "); the results of the passes since the last check "
                               "are invalid (NaN)");
}

extern "C" int64_t rr_tile_schedule(int scan, int pass, int64_t B, int64_t L, int64_t D, int64_t seg, int dtype,
                                    int32_t* tile_k, int32_t* tile_grp, int64_t* max_ckpt_row, int64_t cap) {
  const int64_t T = rr::chunk_len(L, seg);
  if (B <= 0 || L <= 0 || D <= 0 || T == 0 || !rr::valid_dtype(dtype) || (pass != 0 && pass != 1) ||
      scan < 0 || scan > 2) {
    rr::fail(RR_EINVAL, "rr_tile_schedule: invalid arguments");
    return -1;
  }
  const rr::tiles::Geometry g = scan == 2 ? rr::rotlru_geometry(L, D) : rr::rglru_geometry(L, D, dtype, pass, scan == 1);
  const int64_t nGrp = B * g.G, n = nGrp * g.K;
  if (n >= ((int64_t)1 << 31)) {
    rr::fail(RR_EUNSUPPORTED, "rr_tile_schedule: too many tiles");
    return -1;
  }
  if (cap < n || tile_k == nullptr || tile_grp == nullptr) return n;
  const int64_t nC = L / T;
  int64_t worst = -1;
  for (int64_t t = 0; t < n; ++t) {
    const rr::tiles::TileOfTicket tt = rr::tiles::tile_of_ticket((int)t, (int)nGrp, g.K, pass == 1);
    tile_k[t] = tt.k;
    tile_grp[t] = tt.grp;
    if (pass == 1) {
      const int64_t b = tt.grp / g.G;
      for (int w = 0; w < g.NW; ++w) {
        const int row = rr::tiles::bwd_ckpt_row(tt.k * g.NW * g.U + w * g.U, (int)T, (int)L);
        if (row >= 0) worst = std::max<int64_t>(worst, b * nC + row);
      }
    }
  }
  if (max_ckpt_row != nullptr) *max_ckpt_row = worst;
  return n;
}
