// rr_abi.hip — library-wide C entry points: ABI version, error channel and the
// shared shape rules.
#include "rr_common.h"

#include <string>

namespace rr {

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
