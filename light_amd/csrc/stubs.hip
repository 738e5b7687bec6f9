// stubs.hip -- entry points not yet implemented on the GPU.
#include "internal.hpp"
namespace hq {
size_t int4_ws_bytes(int64_t, int64_t, int) { return 0; }
int launch_int4_dequant(const uint32_t *, const float *, const float *, void *, int, int64_t, int64_t, int, int64_t, hipStream_t) {
  return fail(HQ_EUNSUPPORTED, "int4_dequant", "not built");
}
int launch_int4_matmul(const void *, int, const uint32_t *, const float *, const float *, void *, int64_t, int64_t, int64_t, int, void *, hipStream_t) {
  return fail(HQ_EUNSUPPORTED, "int4_matmul", "not built");
}
int launch_moe_q(const void *, const void *, const int64_t *, const int64_t *, int32_t *, int32_t *, const float *, float *, int, int64_t, int64_t, int64_t, int64_t, int64_t, int, int, hipStream_t) {
  return fail(HQ_EUNSUPPORTED, "moe_gemm_q", "not built");
}
}
