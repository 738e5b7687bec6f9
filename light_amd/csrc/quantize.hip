// quantize.hip -- on-GPU q8_1 activation quantizer (q8_1 blocks or the two-level planar act layout).
//
// Block of 32 -> [f16 d][f16 s][i8 q[32]] (quant/q8_1.go:10-18).  Rounding follows
// Light's encodeQ8_0 (quant/quantize.go:70-86): d = amax / 127 (f32), id = 1 / d
// from the unrounded d, q = RoundToEven(v * id); s = f16(f32(sum q) * d).
// Eight lanes own one block (four elements each; act_quant8 in actq.hpp); all
// arithmetic is explicitly rounded so the bytes match the CPU quantizer.
#include "actq.hpp"
#include "internal.hpp"

namespace hq {

template <int XDT>
__device__ __forceinline__ void load4(const void *x, int64_t i, float v[4]) {
  if constexpr (XDT == F32) {
    float4 f = *reinterpret_cast<const float4 *>(static_cast<const float *>(x) + i);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    uint2 u = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(x) + i);
    uint32_t h[4] = {u.x & 0xffffu, u.x >> 16, u.y & 0xffffu, u.y >> 16};
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = XDT == BF16 ? bf2f(h[j]) : h2f(h[j]);
  }
}

template <int XDT, bool ACT>
__global__ __launch_bounds__(256) void quantize_q8_1_kernel(const void *__restrict__ x, uint8_t *__restrict__ dst,
                                                            int64_t nblocks, int64_t q2_off, int64_t d_off,
                                                            int64_t s_off) {
  int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t blk = t >> 3;
  int sub = threadIdx.x & 7;
  bool live = blk < nblocks;
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  if (live) load4<XDT>(x, blk * 32 + sub * 4, v);
  const ActQ q = act_quant8(v);
  if (!live) return;
  if constexpr (ACT) {
    reinterpret_cast<uint32_t *>(dst + blk * 32)[sub] = q.q1;
    reinterpret_cast<uint32_t *>(dst + q2_off + blk * 32)[sub] = q.q2;
    if (sub == 0) {
      reinterpret_cast<float2 *>(dst + d_off)[blk] = make_float2(q.d, q.e);
      reinterpret_cast<float *>(dst + s_off)[blk] = q.sum;
    }
  } else {
    uint8_t *o = dst + blk * 36;
    reinterpret_cast<uint32_t *>(o + 4)[sub] = q.q1;
    if (sub == 0) {
      uint32_t ds = (uint32_t)f2h_rne(q.d) | (uint32_t)f2h_rne(__fmul_rn((float)q.qsum, q.d)) << 16;
      *reinterpret_cast<uint32_t *>(o) = ds;
    }
  }
}

template <bool ACT>
static int launch_q(const void *x, int x_dtype, void *dst, int64_t M, int64_t K, hipStream_t s) {
  int64_t nblocks = M * (K / 32);
  dim3 grid((unsigned)cdiv(nblocks * 8, 256));
  auto *d = static_cast<uint8_t *>(dst);
  int64_t q2off = act_q2_off(M, K), doff = act_d_off(M, K), soff = act_s_off(M, K);
  switch (x_dtype) {
    case F32: quantize_q8_1_kernel<F32, ACT><<<grid, 256, 0, s>>>(x, d, nblocks, q2off, doff, soff); break;
    case BF16: quantize_q8_1_kernel<BF16, ACT><<<grid, 256, 0, s>>>(x, d, nblocks, q2off, doff, soff); break;
    case F16: quantize_q8_1_kernel<F16, ACT><<<grid, 256, 0, s>>>(x, d, nblocks, q2off, doff, soff); break;
    default: return fail(HQ_EUNSUPPORTED, "quantize", "x dtype %d", x_dtype);
  }
  return check_launch("quantize");
}

int launch_quantize_q8_1(const void *x, int x_dtype, void *dst, int64_t M, int64_t K, hipStream_t s) {
  return launch_q<false>(x, x_dtype, dst, M, K, s);
}

int launch_quantize_act(const void *x, int x_dtype, void *dst, int64_t M, int64_t K, hipStream_t s) {
  return launch_q<true>(x, x_dtype, dst, M, K, s);
}

}  // namespace hq
