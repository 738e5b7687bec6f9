// stubs.hip -- entry points not yet implemented on the GPU.
#include "internal.hpp"
namespace hq {
int launch_moe_q(const void *, const void *, const int64_t *, const int64_t *, int32_t *, int32_t *, const float *, float *, int, int64_t, int64_t, int64_t, int64_t, int64_t, int, int, hipStream_t) {
  return fail(HQ_EUNSUPPORTED, "moe_gemm_q", "not built");
}
}
