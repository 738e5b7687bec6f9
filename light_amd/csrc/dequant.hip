// dequant.hip -- bit-exact GGUF block dequantization to F32 / BF16.
//
// Each thread produces eight consecutive outputs (two 16-byte F32 stores or
// one 16-byte BF16 store).  The arithmetic is Light's CPU decoders', operation
// for operation and explicitly rounded, so no multiply-add is fused:
//   Q8_0  y = d * q                         (kernels/cpu/quant_matmul.go:29-34)
//   Q4_0  y = d * (q - 8)                   (kernels/cpu/quant_matmul.go:35-42)
//   Q5_0  y = d * (q5 - 16)                 (kernels/cpu/quant_matmul.go:43-53)
//   Q5_K  y = (d * sc) * q5 - (dmin * m)    (quant/q5_k.go:50-83)
//   Q4_K  y = (d * sc) * q - (dmin * m)     (kernels/cpu/quant_matmul.go:54-68)
//   Q6_K  y = (d * int8 sc) * (raw - 32)    (kernels/cpu/quant_matmul.go:69-87)
//   Q8_1  y = d * q                         (quant/q8_1.go:21-57)
// BF16 rounds the F32 value once (BF16FromF32, dtype/half.go:118-129).
#include "decode.hpp"
#include "internal.hpp"

namespace hq {

template <int DT, int ODT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ w, void *__restrict__ out,
                                                      int64_t n8) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n8) return;
  float y[8];
  decode8<DT>(w, t, y);
  if constexpr (ODT == F32) {
    float4 *o = reinterpret_cast<float4 *>(static_cast<float *>(out) + t * 8);
    o[0] = make_float4(y[0], y[1], y[2], y[3]);
    o[1] = make_float4(y[4], y[5], y[6], y[7]);
  } else {
    uint4 v;
    v.x = f2bf_rne(y[0]) | (uint32_t)f2bf_rne(y[1]) << 16;
    v.y = f2bf_rne(y[2]) | (uint32_t)f2bf_rne(y[3]) << 16;
    v.z = f2bf_rne(y[4]) | (uint32_t)f2bf_rne(y[5]) << 16;
    v.w = f2bf_rne(y[6]) | (uint32_t)f2bf_rne(y[7]) << 16;
    *reinterpret_cast<uint4 *>(static_cast<uint16_t *>(out) + t * 8) = v;
  }
}

template <int DT>
static void launch_dt(const uint8_t *w, void *out, int64_t n, int odt, hipStream_t s) {
  int64_t n8 = n / 8;
  dim3 grid((unsigned)cdiv(n8, 256));
  if (odt == F32)
    dequant_kernel<DT, F32><<<grid, 256, 0, s>>>(w, out, n8);
  else
    dequant_kernel<DT, BF16><<<grid, 256, 0, s>>>(w, out, n8);
}

int launch_dequant(const void *src, void *dst, int64_t n, int src_dtype, int out_dtype, hipStream_t s) {
  auto *w = static_cast<const uint8_t *>(src);
  switch (src_dtype) {
    case Q4_0: launch_dt<Q4_0>(w, dst, n, out_dtype, s); break;
    case Q5_0: launch_dt<Q5_0>(w, dst, n, out_dtype, s); break;
    case Q5_K: launch_dt<Q5_K>(w, dst, n, out_dtype, s); break;
    case Q8_0: launch_dt<Q8_0>(w, dst, n, out_dtype, s); break;
    case Q8_1: launch_dt<Q8_1>(w, dst, n, out_dtype, s); break;
    case Q4_K: launch_dt<Q4_K>(w, dst, n, out_dtype, s); break;
    case Q6_K: launch_dt<Q6_K>(w, dst, n, out_dtype, s); break;
    default: return fail(HQ_EUNSUPPORTED, "dequant", "dtype %d", src_dtype);
  }
  return check_launch("dequant");
}

}  // namespace hq
