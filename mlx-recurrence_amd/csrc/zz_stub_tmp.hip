// temporary: SSD/GLA entry points before their kernels exist
#include "rr_common.h"
extern "C" size_t rr_ssd_workspace_bytes(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int) { return 0; }
extern "C" int rr_ssd_fwd(const void*, const void*, const void*, const void*, const float*, int, int64_t, int64_t L, int64_t, int64_t Dh, int64_t, int64_t seg, const float*, float*, float*, void*, size_t, void*) { if (int rc = rr::check_segment_shape(L, seg, Dh, "Dh")) return rc; return rr::fail(RR_EUNSUPPORTED, "ssd not built yet"); }
extern "C" int rr_ssd_bwd(const float*, const float*, const void*, const void*, const void*, const void*, const float*, int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, const float*, const float*, void*, void*, void*, void*, float*, float*, void*, size_t, void*) { return rr::fail(RR_EUNSUPPORTED, "ssd not built yet"); }
extern "C" size_t rr_gla_workspace_bytes(int64_t, int64_t, int64_t, int64_t, int64_t, int) { return 0; }
extern "C" int rr_gla_fwd(const void*, const void*, const void*, const void*, int, int64_t, int64_t L, int64_t, int64_t Dh, int64_t seg, const float*, float*, float*, void*, size_t, void*) { if (int rc = rr::check_segment_shape(L, seg, Dh, "Dh")) return rc; return rr::fail(RR_EUNSUPPORTED, "gla not built yet"); }
extern "C" int rr_gla_bwd(const float*, const float*, const void*, const void*, const void*, const void*, int, int64_t, int64_t, int64_t, int64_t, int64_t, const float*, const float*, void*, void*, void*, void*, float*, void*, size_t, void*) { return rr::fail(RR_EUNSUPPORTED, "gla not built yet"); }
